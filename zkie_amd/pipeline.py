"""Device-resident commitment pipelines for the synthetic workloads.

commit_round  <- one WHIR round's encode + commit: p3-whir
                 src/pcs/committer/writer.rs:21-86 (Suffix order: the table
                 as coefficient rows of width 2^k, zero-padded by the blowup,
                 dft_batch per column, Merkle commit of the codeword rows)
fold          <- the row fold of p3-whir src/pcs/prover/mod.rs:257-290 and the
                 table fold over the low k variables (common/mle.rs:25-38)
round loop    <- WhirProver::round (prover/mod.rs:196-328) with seeded
                 challenges: k sumcheck rounds over the table times the
                 sumcheck's running weights (compute_sumcheck_polynomials,
                 mod.rs:309-315, with the rules of common/sumcheck.rs:33-89),
                 which leave the table (and the weights) folded over its low k
                 variables; encode + commit the folded table, answer
                 out-of-domain samples on it (mod.rs:226-236), open the
                 previous codeword at STIR indices and fold the opened rows
                 with the round's challenges (mod.rs:247-290), then batch the
                 out-of-domain claims (evaluation constraints) and the STIR
                 claims (selection constraints at w_N^index) with the powers of
                 a seeded gamma into the weights of the next round's sumcheck
                 (mod.rs:292-306); the first sumcheck weighs one seeded
                 evaluation constraint, standing for the initial statement
run_workload  <- the five workloads of zkie_amd.configs, everything in HBM;
                 only roots, requested openings and checks leave the device.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import _native as N
from .configs import (P, SEED_CHALLENGES, SEED_DATA, SEED_GAMMA, SEED_OOD, SEED_QUERIES, SEED_WEIGHTS,
                      Workload, XorShift64, challenges, ef_pow2_chain, query_indices)
from .pcs import (HipMerkleTree, HipMerkleTreeMmcs, constraint_weights, eq_table, fold_rows_at, fold_rows_device,
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
    weight_point: np.ndarray | None = None  # first round: EF point of the initial evaluation constraint
    sumcheck_polys: np.ndarray | None = None  # (k, 3, 2) round polynomials that folded the table
    gamma: np.ndarray | None = None          # EF challenge batching this round's constraint
    stir_points: np.ndarray | None = None    # (q, 2) EF selection points w_N^index of the STIR claims
    claim: np.ndarray | None = None          # sum_j gamma^j ood_j + sum_k gamma^(m+k) stir_k (EF)
    weights: DeviceBuffer | None = None      # the next sumcheck's weights (folded + this constraint)


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


def _batch_claims(claims, gamma) -> np.ndarray:
    """sum_c gamma^c claim_c in EF = F[x]/(x^2 - 7), claims in constraint order."""
    acc0 = acc1 = 0
    g0, g1 = 1, 0
    c0, c1 = int(gamma[0]) % P, int(gamma[1]) % P
    for v in claims:
        v0, v1 = int(v[0]) % P, int(v[1]) % P
        acc0 = (acc0 + g0 * v0 + 7 * g1 * v1) % P
        acc1 = (acc1 + g0 * v1 + g1 * v0) % P
        g0, g1 = (g0 * c0 + 7 * g1 * c1) % P, (g0 * c1 + g1 * c0) % P
    return np.array([acc0, acc1], np.uint64)


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
        g_w, g_gamma = XorShift64(SEED_WEIGHTS), XorShift64(SEED_GAMMA)
        table, t_rows, ext = d_in, wl.rows, False
        t_vars0 = (t_rows.bit_length() - 1) + k
        zw = np.array([g_w.field(), g_w.field()], np.uint64)
        w_point = ef_pow2_chain(zw, t_vars0)
        weights = eq_table(w_point, stream)
        for r in range(wl.rounds):
            chr_ = ch[k * r:k * (r + 1)]
            # k sumcheck rounds fold the table (t_rows x 2^k entries) and its
            # weights over the low k variables
            t_vars = (t_rows.bit_length() - 1) + k
            polys, folded, folded_w = sumcheck_prove(table, ext, weights, t_vars, chr_, stream)
            out.tables.append((folded, t_rows))
            prev = out.rounds[-1]
            table, ext = folded, True
            n_vars = (t_rows.bit_length() - 1)  # the folded table holds t_rows EF entries
            t_rows = t_rows >> k  # EF table of t_rows entries -> rows of 2^k EF
            rnd = commit_round(folded, t_rows, 2 << k, wl.log_blowup, mmcs, stream=stream)
            rnd.sumcheck_polys = polys
            if r == 0:
                rnd.weight_point = w_point
            eq_pts = []
            for _ in range(2):
                z = np.array([g_ood.field(), g_ood.field()], np.uint64)
                rnd.ood_points.append(z)
                eq_pts.append(ef_pow2_chain(z, n_vars))
                rnd.ood_answers.append(mle_eval(folded, n_vars, True, eq_pts[-1], stream))
            sel_pts = np.zeros((0, 2), np.uint64)
            if wl.queries:
                rnd.stir_indices = query_indices(wl.queries, prev.rows, g_stir)
                rnd.stir_folds = fold_rows_at(prev.codeword, prev.rows, k, r > 0, rnd.stir_indices, chr_,
                                              stream)
                # the fold of row i of an N-row codeword is the folded table's
                # polynomial at w_N^i: a selection constraint at that point
                w_n = pow(7, (P - 1) // prev.rows, P)
                sel_pts = np.array([[pow(w_n, int(i), P), 0] for i in rnd.stir_indices], np.uint64)
                rnd.stir_points = sel_pts
            # the round's batched constraint joins the folded weights
            gamma = np.array([g_gamma.field(), g_gamma.field()], np.uint64)
            rnd.gamma = gamma
            claims = [a for a in rnd.ood_answers] + ([f for f in rnd.stir_folds] if wl.queries else [])
            rnd.claim = _batch_claims(claims, gamma)
            weights = constraint_weights(np.array(eq_pts, np.uint64), sel_pts, gamma, n_vars, d_w=folded_w,
                                         accumulate=True, stream=stream)
            rnd.weights = weights
            out.rounds.append(rnd)
    if with_openings and wl.queries:
        g = XorShift64(SEED_QUERIES)
        for rnd in out.rounds:
            open_round(rnd, mmcs, wl.queries, g)
    return out
