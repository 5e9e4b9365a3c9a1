"""Bundle geometry of the q4nx MoE path, parameterised by the layer shape.

Mirrors the constants of ``kernels/moe/pack.py:40-87`` (reference model: H=2560,
I=1088, 128 routed + 1 shared, top-6) as functions of ``(hidden, inter)`` so the
BASELINE shapes (H=2048, I=768, top-8) and the reference model share one code
path.  Per expert: gate+up is one ``[2I, H]`` q4nx matrix (gate rows then up rows),
down is ``[H, Ipad]`` with ``Ipad = ceil(I/256)*256`` and zero input columns past I.
"""

from __future__ import annotations

from dataclasses import dataclass

K_TILE = 256
CHUNK_ROWS = 128
BITS_PER_WEIGHT = 5


def q4nx_bytes(m: int, k: int) -> int:
    """pack_gemv size of an ``[m, k]`` matrix (5 bits per weight, ``quant/q4nx.py:27-28``)."""
    return m * k * BITS_PER_WEIGHT // 8


@dataclass(frozen=True)
class MoeGeometry:
    hidden: int
    inter: int
    n_routed: int = 128
    n_shared: int = 1
    top_k: int = 8

    def __post_init__(self):
        if self.hidden % K_TILE:
            raise ValueError(f"hidden ({self.hidden}) must be a multiple of {K_TILE}")
        if (2 * self.inter) % CHUNK_ROWS:
            raise ValueError(f"2*inter ({2 * self.inter}) must be a multiple of {CHUNK_ROWS}")
        if not 1 <= self.top_k <= min(16, self.n_routed):
            raise ValueError("top_k must be in 1..min(16, n_routed)")
        if self.n_shared not in (0, 1):
            raise ValueError("n_shared must be 0 or 1")

    @property
    def inter_pad(self) -> int:
        return -(-self.inter // K_TILE) * K_TILE

    @property
    def n_experts(self) -> int:
        return self.n_routed + self.n_shared

    @property
    def shared_id(self) -> int:
        """Expert index of the shared expert (``kernels/moe/pack.py:41``: 128 after 0..127)."""
        return self.n_routed

    @property
    def gu_bytes(self) -> int:
        return q4nx_bytes(2 * self.inter, self.hidden)

    @property
    def dn_bytes(self) -> int:
        return q4nx_bytes(self.hidden, self.inter_pad)

    @property
    def expert_bytes(self) -> int:
        return self.gu_bytes + self.dn_bytes

    @property
    def router_bytes(self) -> int:
        return self.n_routed * self.hidden * 2

    def decode_bytes(self, with_shared: bool = True) -> int:
        """Algorithmic HBM bytes of one decode token-layer: router + k (+1) experts."""
        return self.router_bytes + (self.top_k + (1 if with_shared and self.n_shared else 0)) * self.expert_bytes

    @property
    def flops_per_assignment(self) -> int:
        """FLOPs of one (token, expert) pair: 2*H*2I + 2*I*H."""
        return 2 * self.hidden * 2 * self.inter + 2 * self.inter * self.hidden


BASELINE = MoeGeometry(hidden=2048, inter=768, n_routed=128, n_shared=1, top_k=8)
RAON_1_MINI = MoeGeometry(hidden=2560, inter=1088, n_routed=128, n_shared=1, top_k=6)
