#!/usr/bin/env python3
"""Write the golden fixtures of tests/golden/ from the CPU oracle.

  python tests/golden/make_golden.py [--full]

known_answers.json: published vectors (Xoshiro256++, SplitMix64) and small
  oracle outputs: Poseidon2 constants and permutations, leaf hashes,
  compressions, DFTs, folds.
workloads.json (--full): every workload of zkie_amd.configs at its full size
  run through the oracle: the Merkle root of each committed round, checksums
  (sum v_i z^i mod p) of the folded outputs, and the opened indices with the
  first opened row and its authentication path. The largest workload takes
  the oracle about ten minutes on 8 cores.
The reference ships no Goldilocks golden vectors of its own, so apart from the
published PRNG vectors these fixtures freeze the oracle (a restatement of the
reference CPU path) for comparison with the GPU.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402
from zkie_amd import configs as C  # noqa: E402


def hexs(a):
    return [f"{int(x):016x}" for x in np.asarray(a, np.uint64).reshape(-1)]


def known_answers():
    out = {}
    r = O.Xoshiro256pp(state=[1, 2, 3, 4])
    out["xoshiro256pp_state_1_2_3_4"] = [r.next_u64() for _ in range(10)]
    out["splitmix64_seed_0"] = [f"{x:016x}" for x in O.splitmix64(0, 3)]
    a, b, c, d = O.p2_constants()
    out["p2_constants"] = {"rc_init": hexs(a), "rc_final": hexs(b), "rc_internal": hexs(c),
                           "diag15": f"{d:016x}"}
    perms = {}
    for name, st in [("zeros", [0] * 16), ("iota", list(range(16))), ("p_minus_1", [O.P - 1] * 16),
                     ("uniform_seed_3", [int(x) for x in O.gen_uniform(3, 16)])]:
        perms[name] = {"in": hexs(st), "out": hexs(O.p2_permute(st))}
    out["p2_permute"] = perms
    leaves = {}
    for w in (1, 7, 8, 9, 16, 32, 128):
        row = O.gen_uniform(100 + w, w)
        leaves[str(w)] = {"row": hexs(row), "digest": hexs(O.leaf_hash(row))}
    out["leaf_hash"] = leaves
    l, rr = O.gen_uniform(5, 8), O.gen_uniform(6, 8)
    out["compress"] = {"left": hexs(l), "right": hexs(rr), "out": hexs(O.compress(l, rr))}
    dfts = {}
    for lg, w in ((4, 1), (6, 3)):
        x = O.gen_uniform(lg, (1 << lg) * w).reshape(1 << lg, w)
        dfts[f"{lg}x{w}"] = {"in": hexs(x), "out": hexs(O.dft_batch(x))}
    out["dft"] = dfts
    m = O.gen_uniform(40, 4 * 16).reshape(4, 16)
    r4 = C.challenges(4)
    out["fold_k4"] = {"rows": hexs(m), "r": hexs(r4), "out": hexs(O.fold_rows(m, 4, r4, False))}
    return out


def workload(number: int):
    wl = C.CONFIGS[number]
    t0 = time.time()
    gen = {C.GEN_UNIFORM: O.gen_uniform, C.GEN_I16: O.gen_i16, C.GEN_I8: O.gen_i8,
           C.GEN_GAUSS_I16: O.gen_gauss_i16}[wl.kind]
    data = gen(C.SEED_DATA, wl.elems).reshape(wl.rows, wl.cols)
    res = {"name": wl.name, "input_checksum": f"{O.checksum(data):016x}", "rounds": []}
    g = C.XorShift64(C.SEED_QUERIES)

    def commit(coeff):
        cw = O.lde_batch(coeff, wl.log_blowup)
        layers, root = O.merkle_commit(cw)
        rnd = {"rows": cw.shape[0], "width": cw.shape[1], "root": hexs(root),
               "codeword_checksum": f"{O.checksum(cw):016x}"}
        if wl.queries:
            idx = C.query_indices(wl.queries, cw.shape[0], g)
            rnd["queries"] = [int(i) for i in idx]
            rnd["first_row"] = hexs(cw[int(idx[0])])
            rnd["first_path"] = hexs(O.merkle_open(layers, cw.shape[0], int(idx[0])))
            rnd["pruned_count"] = int(O.merkle_open_pruned(layers, cw.shape[0], idx).shape[0])
        return cw, rnd

    cw, rnd = commit(data)
    res["rounds"].append(rnd)
    k = wl.fold_k
    if k and wl.rounds == 0:
        f = O.fold_rows(cw, k, C.challenges(k), False)
        res["fold_checksum"] = f"{O.checksum(f):016x}"
    del cw
    if wl.rounds:
        ch = C.challenges(k * wl.rounds)
        table, ext = data, False
        res["table_checksums"] = []
        for r in range(wl.rounds):
            folded = O.fold_rows(table, k, ch[k * r:k * (r + 1)], ext)
            res["table_checksums"].append(f"{O.checksum(folded):016x}")
            coeff = folded.reshape(-1, 2 << k)
            _, rnd = commit(coeff)
            res["rounds"].append(rnd)
            table, ext = coeff, True
    res["oracle_seconds"] = round(time.time() - t0, 1)
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--full", action="store_true", help="also run the full-size workloads")
    ap.add_argument("--only", type=int, nargs="*", help="workload numbers (with --full)")
    args = ap.parse_args()
    O.set_threads(os.cpu_count() or 1)
    with open(os.path.join(HERE, "known_answers.json"), "w") as f:
        json.dump(known_answers(), f, indent=1)
    if args.full:
        path = os.path.join(HERE, "workloads.json")
        allres = json.load(open(path)) if os.path.exists(path) else {}
        for n in args.only or sorted(C.CONFIGS):
            print(f"workload {n} ...", flush=True)
            allres[str(n)] = workload(n)
            print(f"  done in {allres[str(n)]['oracle_seconds']} s", flush=True)
            with open(path, "w") as f:
                json.dump(allres, f, indent=1)


if __name__ == "__main__":
    main()
