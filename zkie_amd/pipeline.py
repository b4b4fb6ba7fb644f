"""Device-resident commitment pipelines for the synthetic workloads.

commit_round  <- one WHIR round's encode + commit: p3-whir
                 src/pcs/committer/writer.rs:21-86 (Suffix order: the table
                 as coefficient rows of width 2^k, zero-padded by the blowup,
                 dft_batch per column, Merkle commit of the codeword rows)
fold          <- the row fold of p3-whir src/pcs/prover/mod.rs:257-290 and the
                 table fold over the low k variables (common/mle.rs:25-38)
round loop    <- WhirProver::round (prover/mod.rs:196-300) with seeded
                 challenges: k sumcheck rounds over the table times the
                 weight table of one seeded evaluation constraint
                 (compute_sumcheck_polynomials, mod.rs:309-315, with the rules
                 of common/sumcheck.rs:33-89), which leave the table folded
                 over its low k variables; encode + commit the folded table,
                 answer out-of-domain samples on it (mod.rs:226-236), then
                 open the previous codeword at STIR indices and fold the opened
                 rows with the round's challenges (mod.rs:247-290)
run_workload  <- the five workloads of zkie_amd.configs, everything in HBM;
                 only roots, requested openings and checks leave the device.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import _native as N
from .configs import (SEED_CHALLENGES, SEED_DATA, SEED_OOD, SEED_QUERIES, SEED_WEIGHTS, Workload,
                      XorShift64, challenges, ef_pow2_chain, query_indices)
from .pcs import (HipMerkleTree, HipMerkleTreeMmcs, eq_table, fold_rows_at, fold_rows_device,
                  mle_eval, sumcheck_prove)
from ._native import DeviceBuffer


@dataclass
class RoundOutput:
    rows: int                       # codeword rows
    width: int                      # codeword width in base elements
    codeword: DeviceBuffer
    tree: HipMerkleTree
    queries: np.ndarray | None = None
    opened_rows: np.ndarray | None = None
    paths: np.ndarray | None = None
    pruned: np.ndarray | None = None
    ood_points: list = field(default_factory=list)   # EF z of each out-of-domain sample
    ood_answers: list = field(default_factory=list)  # table evaluations at z^(2^i)
    stir_indices: np.ndarray | None = None  # rows of the previous codeword opened this round
    stir_folds: np.ndarray | None = None    # their row folds with this round's challenges
    weight_point: np.ndarray | None = None  # EF point of the sumcheck's evaluation constraint
    sumcheck_polys: np.ndarray | None = None  # (k, 3, 2) round polynomials that folded the table


@dataclass
class WorkloadOutput:
    rounds: list = field(default_factory=list)
    fold: DeviceBuffer | None = None   # row fold of round 0's codeword (configs with fold_k)
    fold_rows: int = 0
    tables: list = field(default_factory=list)  # folded tables (config 5), EF flattened


def commit_round(d_coeffs: DeviceBuffer, h: int, w: int, log_blowup: int,
                 mmcs: HipMerkleTreeMmcs, d_codeword: DeviceBuffer | None = None,
                 stream=None) -> RoundOutput:
    n = h << log_blowup
    tree = mmcs.lde_commit_device(d_coeffs, h, w, log_blowup, d_codeword, stream=stream)
    return RoundOutput(n, w, tree.d_mat, tree)


def open_round(rnd: RoundOutput, mmcs: HipMerkleTreeMmcs, count: int, g: XorShift64):
    idx = query_indices(count, rnd.rows, g)
    rnd.queries = idx
    rnd.opened_rows, rnd.paths = mmcs.open_batches(idx, rnd.tree)
    _, rnd.pruned = mmcs.open_multi_batch(idx, rnd.tree)


def workload_inputs(wl: Workload) -> np.ndarray:
    return N.gen_inputs(SEED_DATA, wl.elems, wl.kind).reshape(wl.rows, wl.cols)


def run_workload(wl: Workload, d_in: DeviceBuffer, with_openings: bool = True,
                 stream=None) -> WorkloadOutput:
    """Run one workload on an input already resident in HBM."""
    mmcs = HipMerkleTreeMmcs()
    out = WorkloadOutput()
    r0 = commit_round(d_in, wl.rows, wl.cols, wl.log_blowup, mmcs, stream=stream)
    out.rounds.append(r0)
    k = wl.fold_k
    if k and wl.rounds == 0:
        # one fold round over the codeword rows (2^k = width)
        ch = challenges(k)
        out.fold = DeviceBuffer(2 * r0.rows)
        out.fold_rows = r0.rows
        fold_rows_device(r0.codeword, r0.rows, k, ch, False, out.fold, stream=stream)
    if wl.rounds:
        ch = challenges(k * wl.rounds)
        g_ood, g_stir = XorShift64(SEED_OOD), XorShift64(SEED_QUERIES + 100)
        g_w = XorShift64(SEED_WEIGHTS)
        table, t_rows, ext = d_in, wl.rows, False
        for r in range(wl.rounds):
            chr_ = ch[k * r:k * (r + 1)]
            # k sumcheck rounds fold the table (t_rows x 2^k entries) over its
            # low k variables
            t_vars = (t_rows.bit_length() - 1) + k
            zw = np.array([g_w.field(), g_w.field()], np.uint64)
            w_point = ef_pow2_chain(zw, t_vars)
            polys, folded, _ = sumcheck_prove(table, ext, eq_table(w_point, stream), t_vars, chr_, stream)
            out.tables.append((folded, t_rows))
            prev = out.rounds[-1]
            table, ext = folded, True
            n_vars = (t_rows.bit_length() - 1)  # the folded table holds t_rows EF entries
            t_rows = t_rows >> k  # EF table of t_rows entries -> rows of 2^k EF
            rnd = commit_round(folded, t_rows, 2 << k, wl.log_blowup, mmcs, stream=stream)
            rnd.weight_point, rnd.sumcheck_polys = w_point, polys
            for _ in range(2):
                z = np.array([g_ood.field(), g_ood.field()], np.uint64)
                rnd.ood_points.append(z)
                rnd.ood_answers.append(mle_eval(folded, n_vars, True, ef_pow2_chain(z, n_vars), stream))
            if wl.queries:
                rnd.stir_indices = query_indices(wl.queries, prev.rows, g_stir)
                rnd.stir_folds = fold_rows_at(prev.codeword, prev.rows, k, r > 0, rnd.stir_indices, chr_,
                                              stream)
            out.rounds.append(rnd)
    if with_openings and wl.queries:
        g = XorShift64(SEED_QUERIES)
        for rnd in out.rounds:
            open_round(rnd, mmcs, wl.queries, g)
    return out
