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


class PagedPQCache:
    """A PQ cache (uniform width) kept in pages: each (batch, head) stream's
    positions live in pages of page_tokens vectors, found through a device
    table of page addresses ([batch * num_heads, max_pages] int64), which is
    what pqkv_encode_paged / pqkv_decode_attn_paged / pqkv_prefill_attn_paged
    take. The cache grows by whole page groups (page p of every stream, one
    allocation [B, H, page_tokens, vector_bytes]) and by rewriting the small
    table, never by copying the tokens it holds; the reference's cache
    concatenates the whole cache on every append
    (src/polarquant_kv_cuda/inference/kv_cache.py:93-112). Keys may carry
    QJL sign pages beside their block pages (same page index)."""

    def __init__(self, batch: int, num_heads: int, head_dim: int, n_bits: int, codebooks, device,
                 page_tokens: int = 256, jl_dim: int = 0, max_pages: int = 16):
        import torch
        if page_tokens < 64 or page_tokens > 65536 or page_tokens & (page_tokens - 1):
            raise ValueError(f"page_tokens must be a power of two in 64..65536, got {page_tokens}")
        self.batch, self.num_heads, self.head_dim, self.n_bits = batch, num_heads, head_dim, int(n_bits)
        self.page_tokens, self.jl_dim = page_tokens, jl_dim
        self.codebooks = codebooks
        self.device = torch.device(device)
        self.seq_len = 0
        self.groups: list = []        # page group p: uint8 [B, H, page_tokens, vector_bytes]
        self.sign_groups: list = []   # with jl_dim: uint8 [B, H, page_tokens, jl_dim / 8]
        self.max_pages = max(1, int(max_pages))
        n = batch * num_heads
        self.table = torch.zeros(n, self.max_pages, dtype=torch.int64, device=self.device)
        self.sign_table = torch.zeros_like(self.table) if jl_dim else None
        self._adopted = None          # (capacity, storage) of caller-managed pages

    def adopt(self, table, capacity: int, storage, sign_table=None) -> None:
        """Use caller-managed pages instead of page groups: table (and, for a
        key cache with signs, sign_table) [batch * num_heads, max_pages]
        int64 device addresses of 16-byte aligned pages covering `capacity`
        positions per stream; storage: the tensors that hold the pages
        (kept alive with the cache). Such a cache does not grow."""
        n = self.batch * self.num_heads
        if table.dim() != 2 or table.shape[0] != n or table.dtype.is_floating_point:
            raise ValueError(f"table must be [{n}, max_pages] int64")
        if capacity > table.shape[1] * self.page_tokens:
            raise ValueError("the table has fewer pages than capacity needs")
        if (sign_table is None) != (self.jl_dim == 0):
            raise ValueError("a sign table goes with jl_dim > 0, and only then")
        self.table, self.sign_table = table, sign_table
        self.max_pages = table.shape[1]
        self.groups, self.sign_groups = [], []
        self._adopted = (int(capacity), storage)

    @property
    def mixed(self) -> bool:
        return False

    @property
    def vector_bytes(self) -> int:
        return vector_bytes(self.head_dim, self.n_bits)

    @property
    def capacity(self) -> int:
        """Positions the allocated pages hold."""
        if self._adopted is not None:
            return self._adopted[0]
        return len(self.groups) * self.page_tokens

    @property
    def qjl_signs(self):
        """Stands for the sign array of PQCache: not None when the cache keeps signs."""
        return self.sign_table

    def head_bits(self) -> list:
        return [self.n_bits] * self.num_heads

    def _widen(self, pages: int) -> None:
        import torch
        width = self.max_pages
        while width < pages:
            width *= 2
        if width == self.max_pages:
            return
        n = self.batch * self.num_heads
        t = torch.zeros(n, width, dtype=torch.int64, device=self.device)
        t[:, :self.max_pages] = self.table
        self.table = t
        if self.sign_table is not None:
            t = torch.zeros_like(self.table)
            t[:, :self.max_pages] = self.sign_table
            self.sign_table = t
        self.max_pages = width

    def ensure(self, positions: int) -> None:
        """Allocate page groups until `positions` positions fit."""
        import torch
        if self._adopted is not None:
            if positions > self._adopted[0]:
                raise ValueError(f"{positions} positions exceed the adopted pages' {self._adopted[0]}")
            return
        need = -(-int(positions) // self.page_tokens)
        if need <= len(self.groups):
            return
        self._widen(need)
        B, H, P = self.batch, self.num_heads, self.page_tokens
        streams = torch.arange(B * H, dtype=torch.int64, device=self.device)
        while len(self.groups) < need:
            p = len(self.groups)
            g = torch.zeros(B, H, P, self.vector_bytes, dtype=torch.uint8, device=self.device)
            self.groups.append(g)
            self.table[:, p] = g.data_ptr() + streams * (P * self.vector_bytes)
            if self.sign_table is not None:
                sg = torch.zeros(B, H, P, self.jl_dim // 8, dtype=torch.uint8, device=self.device)
                self.sign_groups.append(sg)
                self.sign_table[:, p] = sg.data_ptr() + streams * (P * (self.jl_dim // 8))

    def memory_bytes(self) -> int:
        """Device bytes of the allocated pages (and the page tables)."""
        n = sum(g.numel() for g in self.groups) + sum(g.numel() for g in self.sign_groups)
        n += self.table.numel() * 8 + (self.sign_table.numel() * 8 if self.sign_table is not None else 0)
        return n

    def to_contiguous(self, length: int | None = None) -> "PQCache":
        """The first `length` (default seq_len) positions as a PQCache
        ([B, H, length, vector_bytes]; with signs when the cache keeps them).
        A copy: for checks and for callers that need one contiguous array."""
        import torch
        if self._adopted is not None:
            raise ValueError("a cache on caller-managed pages is gathered by its owner")
        S = self.seq_len if length is None else int(length)
        P, vb = self.page_tokens, self.vector_bytes
        B, H = self.batch, self.num_heads
        n = -(-S // P)
        blocks = torch.cat(self.groups[:n], dim=2)[:, :, :S].contiguous() if n else \
            torch.zeros(B, H, 0, vb, dtype=torch.uint8, device=self.device)
        signs = None
        if self.sign_table is not None:
            signs = torch.cat(self.sign_groups[:n], dim=2)[:, :, :S].contiguous() if n else \
                torch.zeros(B, H, 0, self.jl_dim // 8, dtype=torch.uint8, device=self.device)
        return PQCache(blocks=blocks, head_dim=self.head_dim, n_bits=self.n_bits, seq_len=S, max_seq_len=S,
                       codebooks=self.codebooks, qjl_signs=signs, jl_dim=self.jl_dim)

    def select_batch(self, index) -> None:
        """Reorder / select / repeat the batch rows (beam search): every page
        group is gathered along the batch dimension (index: device int64)."""
        import torch
        if self._adopted is not None:
            raise ValueError("a cache on caller-managed pages is reordered by its owner")
        self.groups = [g.index_select(0, index) for g in self.groups]
        self.sign_groups = [g.index_select(0, index) for g in self.sign_groups]
        self.batch = int(index.numel())
        n = self.batch * self.num_heads
        self.table = torch.zeros(n, self.max_pages, dtype=torch.int64, device=self.device)
        self.sign_table = torch.zeros_like(self.table) if self.jl_dim else None
        streams = torch.arange(n, dtype=torch.int64, device=self.device)
        P = self.page_tokens
        for p, g in enumerate(self.groups):
            self.table[:, p] = g.data_ptr() + streams * (P * self.vector_bytes)
        for p, g in enumerate(self.sign_groups):
            self.sign_table[:, p] = g.data_ptr() + streams * (P * (self.jl_dim // 8))


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
