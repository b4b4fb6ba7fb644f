"""Independent pure-Python restatement of the commitment path (small inputs only).

TEST INFRASTRUCTURE ONLY. It is written in a different form from the C
oracle so that the two check each other:
  * Poseidon2 follows the addition chains of poseidon2_merkle.cu:63-142
    (apply_mat4 through t01/t23/t0123, halving by multiplying with (p+1)/2),
    while the C oracle uses explicit matrix products and field inverses;
  * the DFT is the O(n^2) definition with python integers;
  * the Merkle tree is built recursively from the layer-length recurrence.
"""
from __future__ import annotations

P = 0xFFFFFFFF00000001
W_EXT = 7
HALF = (P + 1) // 2  # 0x7FFFFFFF80000001, poseidon2_merkle.cu:39


def gen(k: int) -> int:
    return pow(7, (P - 1) >> k, P)


# ---- rand 0.10 SmallRng -------------------------------------------------------
def splitmix64(state: int):
    M = (1 << 64) - 1
    while True:
        state = (state + 0x9E3779B97F4A7C15) & M
        z = state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
        yield z ^ (z >> 31)


class Xoshiro:
    M = (1 << 64) - 1

    def __init__(self, seed: int):
        g = splitmix64(seed)
        self.s = [next(g) for _ in range(4)]

    def next(self) -> int:
        s, M = self.s, self.M
        rotl = lambda x, k: ((x << k) | (x >> (64 - k))) & M
        res = (rotl((s[0] + s[3]) & M, 23) + s[0]) & M
        t = (s[1] << 17) & M
        s[2] ^= s[0]
        s[3] ^= s[1]
        s[1] ^= s[2]
        s[0] ^= s[3]
        s[2] ^= t
        s[3] = rotl(s[3], 45)
        return res

    def field(self) -> int:
        while True:
            x = self.next()
            if x < P:
                return x


def derive_constants():
    r = Xoshiro(1)
    init = [r.field() for _ in range(64)]
    final = [r.field() for _ in range(64)]
    internal = [r.field() for _ in range(22)]
    diag15 = pow(pow(2, 32, P), P - 2, P)
    return init, final, internal, diag15


# ---- Poseidon2 (poseidon2_merkle.cu form) -------------------------------------
def _sbox(x):
    x2 = x * x % P
    x3 = x2 * x % P
    x4 = x2 * x2 % P
    return x3 * x4 % P


def _mat4(x, o):
    t01 = (x[o] + x[o + 1]) % P
    t23 = (x[o + 2] + x[o + 3]) % P
    t0123 = (t01 + t23) % P
    t01123 = (t0123 + x[o + 1]) % P
    t01233 = (t0123 + x[o + 3]) % P
    x0, x2 = x[o], x[o + 2]
    x[o + 3] = (t01233 + 2 * x0) % P
    x[o + 1] = (t01123 + 2 * x2) % P
    x[o] = (t01123 + t01) % P
    x[o + 2] = (t01233 + t23) % P


def _mds(st):
    for o in range(0, 16, 4):
        _mat4(st, o)
    sums = [sum(st[j + k] for j in range(0, 16, 4)) % P for k in range(4)]
    for i in range(16):
        st[i] = (st[i] + sums[i % 4]) % P


def _halve(x, times=1):
    for _ in range(times):
        x = x * HALF % P
    return x


def _internal(st, diag15):
    s = sum(st) % P
    x = st
    out = [0] * 16
    out[0] = (s - 2 * x[0]) % P
    out[1] = (s + x[1]) % P
    out[2] = (s + 2 * x[2]) % P
    out[3] = (s + _halve(x[3])) % P
    out[4] = (s + 3 * x[4]) % P
    out[5] = (s + 4 * x[5]) % P
    out[6] = (s - _halve(x[6])) % P
    out[7] = (s - 3 * x[7]) % P
    out[8] = (s - 4 * x[8]) % P
    out[9] = (s + _halve(x[9], 3)) % P
    out[10] = (s + _halve(x[10], 4)) % P
    out[11] = (s + _halve(x[11], 5)) % P
    out[12] = (s - _halve(x[12], 3)) % P
    out[13] = (s - _halve(x[13], 4)) % P
    out[14] = (s - _halve(x[14], 5)) % P
    out[15] = (s + x[15] * diag15) % P
    st[:] = out


class Poseidon2:
    def __init__(self, consts=None):
        self.init, self.final, self.internal, self.diag15 = consts or derive_constants()

    def permute(self, state):
        st = [int(v) % P for v in state]
        _mds(st)
        for r in range(4):
            st = [_sbox((st[i] + self.init[16 * r + i]) % P) for i in range(16)]
            _mds(st)
        for r in range(22):
            st[0] = _sbox((st[0] + self.internal[r]) % P)
            _internal(st, self.diag15)
        for r in range(4):
            st = [_sbox((st[i] + self.final[16 * r + i]) % P) for i in range(16)]
            _mds(st)
        return st

    def hash_row(self, row):
        """PaddingFreeSponge<Perm,16,8,8>::hash_iter."""
        st = [0] * 16
        row = [int(v) for v in row]
        for pos in range(0, len(row), 8):
            chunk = row[pos:pos + 8]
            st[:len(chunk)] = chunk
            st = self.permute(st)
        return st[:8]

    def compress(self, left, right):
        return self.permute(list(left) + list(right))[:8]


# ---- DFT / fold --------------------------------------------------------------
def dft(col):
    n = len(col)
    k = n.bit_length() - 1
    g = gen(k)
    return [sum(int(c) * pow(g, i * j, P) for j, c in enumerate(col)) % P for i in range(n)]


def ef_mul(a, b):
    return ((a[0] * b[0] + W_EXT * a[1] * b[1]) % P, (a[0] * b[1] + a[1] * b[0]) % P)


def mle_eval_ef(values, point):
    """mle.rs:8-22 with EF values and EF point, LSB-first."""
    buf = [tuple(v) for v in values]
    for p in point:
        buf = [((a[0] + ef_mul(p, ((b[0] - a[0]) % P, (b[1] - a[1]) % P))[0]) % P,
                (a[1] + ef_mul(p, ((b[0] - a[0]) % P, (b[1] - a[1]) % P))[1]) % P)
               for a, b in zip(buf[0::2], buf[1::2])]
    return buf[0]


# ---- Merkle --------------------------------------------------------------------
def padded_len(raw, n=2):
    if raw <= 1:
        return raw
    if raw >= n:
        return -(-raw // n) * n
    return n


def merkle_layers(rows, perm: Poseidon2):
    h = len(rows)
    layer = [perm.hash_row(r) for r in rows] + [[0] * 8] * (padded_len(h) - h)
    layers = [layer]
    while len(layer) > 1:
        nxt = [perm.compress(layer[2 * i], layer[2 * i + 1]) for i in range(len(layer) // 2)]
        nxt += [[0] * 8] * (padded_len(len(nxt)) - len(nxt))
        layers.append(nxt)
        layer = nxt
    return layers
