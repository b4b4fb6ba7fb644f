#!/usr/bin/env python3
"""Benchmark of the shard commitment hot path on one MI355X.

One step = one commitment of the resident input: coset/subgroup LDE (blowup
4), the Poseidon2 Merkle tree over the codeword rows (root read back), and
one fold round (k = 4) over the codeword, on 2^24 rows x 16 columns of
uniform Goldilocks elements (2^28 input elements). Prints one JSON line.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--config N]
                  [--no-cpu-baseline] [--prover-data]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
METRIC = "committed Goldilocks elems/sec (LDE+Merkle) at 2^24x16, % HBM roofline"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-rows", type=int, default=1 << 20,
                    help="coefficient rows of the CPU baseline sample")
    ap.add_argument("--prover-data", action="store_true",
                    help="after the timed steps, also time streaming the committed tree out of "
                         "HBM in the batch-cache prover-data format into a discarding host sink")
    ap.add_argument("--sumcheck", action="store_true",
                    help="after the timed steps, also time the WHIR round's sumcheck (k rounds over "
                         "the 2^22-entry table of the opening-pipeline workload times an eq weight "
                         "table) against the HBM roofline")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="after the run, copy MIB MiB device to device three times (a plain "
                         "copy kernel of known size for scaling rocprofv3 FETCH/WRITE_SIZE)")
    return ap.parse_args()


def cpu_baseline(wl, rows: int, threads: int = 0):
    """The oracle (C restatement of the reference CPU path) on a bounded
    sample of the same workload, on `threads` host threads (0: all host
    cores, at most 16, the CPU share of the machine)."""
    from oracle import oracle as O
    from zkie_amd import configs as C

    threads = threads or min(os.cpu_count() or 1, 16)
    O.set_threads(threads)
    sample = wl.scaled(rows)
    data = O.gen_uniform(C.SEED_DATA, sample.elems).reshape(sample.rows, sample.cols)
    ch = C.challenges(wl.fold_k) if wl.fold_k else None
    t0 = time.perf_counter()
    cw = O.lde_batch(data, sample.log_blowup)
    _, root = O.merkle_commit(cw)
    if ch is not None:
        O.fold_rows(cw, wl.fold_k, ch, False)
    dt = time.perf_counter() - t0
    return {
        "value": sample.elems / dt,
        "unit": "elem/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{sample.rows} rows x {sample.cols} cols, blowup {1 << sample.log_blowup}, "
                  f"LDE + Merkle root + fold k={wl.fold_k}; {dt:.2f} s wall",
    }


# Issue peak of the VALU: 256 CUs x 2.4 GHz x 1.35 wave-instructions per CU
# per clock, the fastest rate measured on gfx950 (plain 32-bit VOP1/VOP2 ops;
# v_mad_u64_u32 and other VOP3 forms issue at about 0.86-0.93).
VALU_PEAK_WINSTR_S = 256 * 2.4e9 * 1.35


def prover_data_stream(N, d_cw, n: int, w: int, d_layers, stream, reps: int = 2):
    """Time zkie_prover_data_write of the step's tree (matrix + digest layers,
    the bytes after the batch-cache header) into a sink that drops every
    piece: the device-to-host rate of the stream, without the sink's own cost
    (a file adds its write rate)."""
    size = N.prover_data_size(n, w)

    def sink(view):
        pass

    N.prover_data_write(d_cw.addr, n, w, d_layers.addr, sink, stream.handle)  # first use
    t0 = time.perf_counter()
    for _ in range(reps):
        N.prover_data_write(d_cw.addr, n, w, d_layers.addr, sink, stream.handle)
    dt = (time.perf_counter() - t0) / reps
    return {"bytes": size, "ms": round(dt * 1e3, 3), "GB_per_s": round(size / dt / 1e9, 2),
            "sink": "discard", "path": "HBM -> pinned staging (2 x 16 MiB) -> host callback"}


def sumcheck_rounds(N, stream, t: int = 22, k: int = 4, reps: int = 20):
    """Time zkie_sumcheck_prove: k rounds over a base table of 2^t entries
    times an EF weight table (the first round of the opening-pipeline
    workload), per kernel with the library's HIP-event timers. Algorithmic
    bytes: round 0's sums read both tables (f: 8 B per base entry, h: 16 B),
    then every round's fold reads both tables (f: 8 B in round 0, then 16 B
    EF) and writes the two halved EF tables, the folds before the last one
    forming the next round's sums in the same pass."""
    import numpy as np

    from zkie_amd import configs as C
    from zkie_amd.pcs import eq_table, sumcheck_prove
    from zkie_amd._native import DeviceBuffer

    d_f = DeviceBuffer.from_array(N.gen_inputs(C.SEED_DATA, 1 << t, 0))  # uniform
    d_h = eq_table(C.ef_pow2_chain(np.array([5, 6], np.uint64), t), stream.handle)
    r = C.challenges(k)
    sumcheck_prove(d_f, False, d_h, t, r, stream.handle)  # first use
    N.check(N.load().zkie_device_synchronize(), "sync")
    N.profile_enable(True)
    N.profile_reset()
    t0 = time.perf_counter()
    for _ in range(reps):
        sumcheck_prove(d_f, False, d_h, t, r, stream.handle)
    dt = (time.perf_counter() - t0) / reps
    kern = {name: N.profile_query(name) for name in ("sumcheck_round", "sumcheck_fold_round", "sumcheck_fold",
                                                  "sumcheck_finish")}
    N.profile_enable(False)
    alg = (1 << t) * (8 + 16)
    for i in range(k):
        m = t - i
        fb = 8 if i == 0 else 16
        alg += (1 << m) * (fb + 16) + (1 << (m - 1)) * 32
    dev_ms = sum(ms for _, ms in kern.values()) / reps
    return {"table": f"2^{t} base x EF weights", "rounds": k, "ms_per_call": round(dt * 1e3, 3),
            "kernel_ms_per_call": round(dev_ms, 3), "alg_bytes": alg,
            "GB_per_s_kernels": round(alg / (dev_ms * 1e-3) / 1e9, 1) if dev_ms else None,
            "hbm_frac_kernels": round(alg / (dev_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4) if dev_ms else None,
            "per_kernel_avg_ms": {n_: round(ms / max(c, 1), 4) for n_, (c, ms) in kern.items()}}


def h2d_seconds(N, d_in, data, reps: int = 2) -> float:
    """Mean time of a synchronous upload of the step's input (8 B per
    element) from pageable host memory into its device buffer."""
    d_in.upload(data)  # first use of these host pages
    N.check(N.load().zkie_device_synchronize(), "sync")
    t0 = time.perf_counter()
    for _ in range(reps):
        d_in.upload(data)
    N.check(N.load().zkie_device_synchronize(), "sync")
    return (time.perf_counter() - t0) / reps


def leaf_profile():
    """Per-launch figures of the leaf kernel measured with rocprofv3 at this
    workload: HBM bytes (FETCH_SIZE + WRITE_SIZE, copy-kernel scaled) and VALU
    wave-instructions, from the committed profile summaries."""
    path = os.path.join(ROOT, "profiles", "p2_leaf_traffic.json")
    if not os.path.exists(path):
        return {}
    with open(path) as f:
        return json.load(f)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for {args.gpus}); the multi-GPU "
              "sharding of this path is a design, not a measured configuration.", file=sys.stderr)
        sys.exit(2)

    from zkie_amd import _native as N
    from zkie_amd import configs as C
    from zkie_amd.pcs import HipMerkleTreeMmcs, fold_rows_device, lde_device
    from zkie_amd._native import DeviceBuffer

    wl = C.CONFIGS[args.config]
    assert N.device_count() >= 1, "no HIP device"
    data = N.gen_inputs(C.SEED_DATA, wl.elems, wl.kind)
    d_in = DeviceBuffer.from_array(data)
    n, w = wl.codeword_rows, wl.cols
    d_cw = DeviceBuffer(n * w)
    lens = N.merkle_layout(n)
    d_layers = DeviceBuffer(sum(lens) * 8)
    d_fold = DeviceBuffer(2 * n) if wl.fold_k else None
    ch = C.challenges(wl.fold_k) if wl.fold_k else None
    mmcs = HipMerkleTreeMmcs()
    L = N.load()
    import numpy as np
    root = np.zeros(8, np.uint64)
    stream = N.Stream()

    def step():
        lde_device(d_in, wl.rows, w, wl.log_blowup, d_cw, stream=stream.handle)
        N.check(L.zkie_merkle_commit(d_cw.addr, n, w, d_layers.addr, N.p(root), stream.handle), "commit")
        if wl.fold_k:
            fold_rows_device(d_cw, n, wl.fold_k, ch, False, d_fold, stream=stream.handle)

    for _ in range(args.warmup):
        step()
    N.check(L.zkie_device_synchronize(), "sync")
    N.profile_enable(True)
    N.profile_reset()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    N.check(L.zkie_device_synchronize(), "sync")
    t = (time.perf_counter() - t0) / args.steps
    per_kernel = {k: N.profile_query(k) for k in N.profile_names()}
    N.profile_enable(False)
    h2d_s = h2d_seconds(N, d_in, data)
    del data

    value = wl.elems / t
    # Dominant kernel: the Merkle leaf hash (2 of the 3 permutations per row).
    leaf_n, leaf_ms = per_kernel.get("p2_leaf", (0, 0.0))
    leaf_avg_ms = leaf_ms / max(leaf_n, 1)
    leaf_alg_bytes = n * w * 8 + n * 64       # read the codeword rows, write layer-0 digests
    achieved = leaf_alg_bytes / (leaf_avg_ms * 1e-3) / 1e9 if leaf_avg_ms else 0.0
    prof = leaf_profile() if args.config == 3 else {}
    traffic = prof.get("bytes_per_launch")
    stage_ms = {k: round(ms / max(cnt, 1) * max(cnt, 1) / args.steps, 3) for k, (cnt, ms) in per_kernel.items()}
    # whole-step HBM floor: 8 B in + 32 B codeword + 32 B digests (+ 36 B fold) per input element
    step_alg_bytes = wl.elems * (72 + (36 if wl.fold_k else 0))
    # Per stage: time per step and its algorithmic HBM bytes at the 8 TB/s peak.
    # LDE: every pass reads and writes the codeword (the first reads the input);
    # Merkle: rows in, every digest layer written once and read once;
    # fold: codeword in, one EF element per row out.
    lg_n = n.bit_length() - 1
    passes = (lg_n + 8) // 9
    lde_bytes = wl.elems * 8 + n * w * 8 * (2 * passes - 1)
    merkle_bytes = n * w * 8 + 2 * (2 * n) * 64
    fold_bytes = n * w * 8 + n * 16 if wl.fold_k else 0

    def stage(names, alg):
        ms = sum(per_kernel.get(k, (0, 0.0))[1] for k in names) / args.steps
        return {"ms": round(ms, 3), "alg_bytes": alg,
                "hbm_frac": round(alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4) if ms else None}

    stages = {"lde": stage([k for k in per_kernel if k.startswith("ntt_pass")], lde_bytes),
              "merkle": stage(["p2_leaf", "p2_compress", "p2_subtree"], merkle_bytes)}
    if wl.fold_k:
        stages["fold"] = stage(["fold_rows"], fold_bytes)

    out = {
        "metric": METRIC,
        "value": value,
        "unit": "elem/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": t * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u64",
        "data": "synthetic",
        "config": {"workload": wl.name, "rows": wl.rows, "cols": wl.cols,
                   "log_blowup": wl.log_blowup, "fold_k": wl.fold_k,
                   "codeword_rows": n, "parallelism": "single-gpu"},
        "roofline": {"bound": "hbm", "kernel": "p2_leaf", "achieved": achieved,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "traffic": traffic, "avg_ms": leaf_avg_ms},
        "step_hbm_frac": step_alg_bytes / t / 1e9 / HBM_PEAK_GBS,
        # The leaf kernel is bound by VALU issue, not HBM: its rocprof VALU count
        # over its live duration against the issue peak.
        "valu_roofline": ({"kernel": "p2_leaf", "achieved": prof["valu_per_launch"] / (leaf_avg_ms * 1e-3),
                           "peak": VALU_PEAK_WINSTR_S, "unit": "wave-instr/s",
                           "frac": prof["valu_per_launch"] / (leaf_avg_ms * 1e-3) / VALU_PEAK_WINSTR_S}
                          if prof.get("valu_per_launch") and leaf_avg_ms else None),
        "stage_ms_per_step": stage_ms,
        "stages": stages,
        # A caller that hands over the input in host memory (the reference's
        # dft_batch takes a host RowMajorMatrix) also pays its upload; the
        # tree stays in HBM and only the root comes back (inside the step).
        "pcie_inclusive": {"value": wl.elems / (t + h2d_s), "unit": "elem/s",
                           "h2d_ms": round(h2d_s * 1e3, 3),
                           "h2d_GB_per_s": round(wl.elems * 8 / h2d_s / 1e9, 2),
                           "source": "pageable host memory (numpy), synchronous copy"},
    }
    if args.prover_data:
        out["prover_data_stream"] = prover_data_stream(N, d_cw, n, w, d_layers, stream)
    if args.sumcheck:
        out["sumcheck"] = sumcheck_rounds(N, stream)
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(wl, args.cpu_rows)
        # single-threaded, on a sample 16x smaller (the reference quotes its GPU
        # speed-up against one CPU thread, whir.rs:55-56)
        out["cpu_baseline_1thread"] = cpu_baseline(wl, max(args.cpu_rows >> 4, 1 << 10), threads=1)
    print(json.dumps(out), flush=True)
    if args.copy_calibration:
        nbytes = args.copy_calibration << 20
        src, dst = DeviceBuffer(nbytes // 8), DeviceBuffer(nbytes // 8)
        for _ in range(3):
            N.check(L.zkie_memcpy_dtod(dst.addr, src.addr, nbytes, None), "copy")
        N.check(L.zkie_device_synchronize(), "sync")
        print(f"copy calibration: 3 device-to-device copies of {nbytes} bytes", file=sys.stderr)


if __name__ == "__main__":
    main()
