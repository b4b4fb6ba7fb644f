"""The synthetic commitment workloads (shapes, generators, seeds).

Seeds: data 0, fold challenges 1, query indices 2, out-of-domain points 3,
the initial evaluation constraint 4, the constraint-batching challenges 5. Inputs come from the
XorShift64 generator of common/field.rs:17-36 (zkie_gen_inputs).
  1  2^16 int16 values, one column, blowup 4 -> 2^18-row codeword, Merkle root.
  2  GPT-2-small 768x3072 weight matrix, Irwin-Hall gaussian int16
     (std 0.02 * 2^12): the first 2^21 values as 2^17 rows x 16 columns,
     blowup 4, root plus 64 opening paths and one pruned multiproof.
  3  2^24 rows x 16 columns of uniform field elements, blowup 4
     (2^26-row codeword), row-wise Merkle tree, one fold round (k = 4).
  4  MoE expert shard: 2^27 int8 values in [-127, 127] as 2^20 rows x 128
     columns, blowup 2, Merkle root.
  5  2^22 uniform field elements, WHIR-shaped with folding factor k = 4 and
     blowup 8: round 0 commits 2^18 x 16 -> 2^21 x 16, then three rounds fold
     the table by 2^4 (EF challenges), re-encode at blowup 8 and commit
     (2^14, 2^10, 2^6 EF rows x 16 EF before blowup), 128 openings per
     commitment.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

GEN_UNIFORM, GEN_I16, GEN_I8, GEN_GAUSS_I16 = 0, 1, 2, 3
SEED_DATA, SEED_CHALLENGES, SEED_QUERIES, SEED_OOD, SEED_WEIGHTS, SEED_GAMMA = 0, 1, 2, 3, 4, 5
P = 0xFFFFFFFF00000001


@dataclass(frozen=True)
class Workload:
    number: int
    name: str
    rows: int          # coefficient rows h
    cols: int          # base-field width w
    log_blowup: int
    kind: int          # input generator
    fold_k: int = 0    # fold rounds use 2^fold_k-wide rows (0 = no fold)
    rounds: int = 0    # WHIR rounds after round 0 (config 5)
    queries: int = 0   # openings per commitment

    @property
    def elems(self) -> int:
        return self.rows * self.cols

    @property
    def codeword_rows(self) -> int:
        return self.rows << self.log_blowup

    def scaled(self, rows: int) -> "Workload":
        """The same workload on fewer coefficient rows (for parity tests)."""
        return Workload(self.number, f"{self.name}@rows={rows}", rows, self.cols, self.log_blowup,
                        self.kind, self.fold_k, self.rounds, self.queries)


CONFIGS = {
    1: Workload(1, "i16_2^16x1_blowup4_root", 1 << 16, 1, 2, GEN_I16),
    2: Workload(2, "gpt2_768x3072_as_2^17x16_blowup4_64paths", 1 << 17, 16, 2, GEN_GAUSS_I16, queries=64),
    3: Workload(3, "uniform_2^24x16_blowup4_root_fold4", 1 << 24, 16, 2, GEN_UNIFORM, fold_k=4),
    4: Workload(4, "moe_int8_2^20x128_blowup2_root", 1 << 20, 128, 1, GEN_I8),
    5: Workload(5, "whir_2^22_blowup8_k4_3rounds_128q", 1 << 18, 16, 3, GEN_UNIFORM, fold_k=4,
                rounds=3, queries=128),
}


class XorShift64:
    """common/field.rs:17-36 (for challenges and query indices)."""

    M = (1 << 64) - 1

    def __init__(self, seed: int):
        self.s = (seed + 0x9E3779B97F4A7C15) & self.M

    def next_u64(self) -> int:
        x = self.s
        x ^= (x << 13) & self.M
        x ^= x >> 7
        x ^= (x << 17) & self.M
        self.s = x
        return x

    def field(self) -> int:
        return self.next_u64() % P


def challenges(count: int, seed: int = SEED_CHALLENGES) -> np.ndarray:
    """`count` EF challenges (c0, c1), each c = field() (uniform mod p)."""
    g = XorShift64(seed)
    return np.array([[g.field(), g.field()] for _ in range(count)], np.uint64)


def ef_pow2_chain(z, n: int) -> np.ndarray:
    """[z, z^2, z^4, ..., z^(2^(n-1))] in EF = F[x]/(x^2 - 7): the coordinates
    of a univariate out-of-domain sample z expanded to n variables, variable 0
    first (p3's Point::expand_from_univariate lists the same powers most
    significant variable first; zkie_mle_eval takes variable 0 first)."""
    out = []
    c0, c1 = int(z[0]) % P, int(z[1]) % P
    for _ in range(n):
        out.append([c0, c1])
        c0, c1 = (c0 * c0 + 7 * c1 * c1) % P, (2 * c0 * c1) % P
    return np.array(out, np.uint64).reshape(n, 2)


def query_indices(count: int, height: int, g: XorShift64) -> np.ndarray:
    """min(count, height) distinct indices in [0, height), sorted ascending,
    following get_challenge_stir_queries (p3-whir src/pcs/utils.rs:70-119):
    draw uniform indices (next_u64() mod height: the low log2(height) bits,
    height being a power of two), keep a draw only if it is new, until the
    target count is reached (count >= height opens every row), then sort."""
    assert height > 0 and height & (height - 1) == 0, "the folded domain size is a power of two"
    target = min(count, height)
    seen: set[int] = set()
    while len(seen) < target:
        seen.add(g.next_u64() % height)
    return np.array(sorted(seen), np.uint64)
