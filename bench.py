#!/usr/bin/env python3
"""Benchmark of the shard commitment hot path on one MI355X.

One step = one commitment of the resident input: the LDE (blowup 4), the
Poseidon2 Merkle tree over the codeword rows (root read back), and one fold
round (k = 4) over the codeword, on 2^24 rows x 16 columns of uniform
Goldilocks elements (2^28 input elements). Prints one JSON line.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--config N]
                  [--no-cpu-baseline] [--prover-data] [--sumcheck]
  python bench.py --valu-peak           # VALU issue rates per instruction kind
  python bench.py --ingest-counters DIR # rocprofv3 counter CSVs -> profile JSON

Rooflines. The step is bound by VALU issue (Poseidon2), not by HBM, so every
roofline is given with both components:
  * HBM: algorithmic bytes (the per-element figures below) over the measured
    time, against 8 TB/s;
  * VALU: VALU wave-instructions (rocprofv3 SQ_INSTS_VALU per launch, from the
    committed counter profile, used only while its source hash matches the
    kernel sources) over the measured time, against the issue peak measured
    live in the same run by the probe kernels of libzkie_valu_probe.so;
  * `bound` names the larger of the two bounds, t_hbm = bytes / 8 TB/s and
    t_valu = instructions / issue peak, and `frac` = t_bound / t_measured.
Algorithmic bytes per input element at the 2^24 x 16 workload: LDE 8 in +
32 codeword out = 40; Merkle 32 (2^27 digests of 64 B written); fold 32
codeword in + 4 out = 36; the step (fused minimum) 108.
"""
from __future__ import annotations

import argparse
import csv
import glob
import hashlib
import json
import os
import platform
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
CLOCK_HZ = 2.4e9               # MI355X peak engine clock
CUS = 256
METRIC = "committed Goldilocks elems/sec (LDE+Merkle) at 2^24x16, % HBM roofline"
COUNTERS_JSON = os.path.join(ROOT, "profiles", "commit_step_counters.json")

# Profiler names of the library's kernels and the stage each belongs to.
# With the last NTT pass fused with the leaf hash (ntt_last_leaf) one kernel
# does part of both the LDE and the Merkle stage; the two are then reported
# as one stage, lde+merkle.
STAGE_KERNELS = {
    "lde": ("ntt_pass_first", "ntt_pass_mid", "ntt_pass_last"),
    "merkle": ("p2_leaf", "p2_compress", "p2_subtree"),
    "lde+merkle": ("ntt_pass_first", "ntt_pass_mid", "ntt_pass_last", "ntt_last_leaf", "p2_leaf",
                   "p2_compress", "p2_subtree"),
    "fold": ("fold_rows",),
}

# VALU probe kinds (zkie_amd/csrc/valu_probe.hip).
PROBE_KINDS = ["v_add_u32 (VOP2)", "v_add_co_u32 (VOP3, SGPR carry)", "v_mad_u64_u32",
               "v_mul_lo_u32", "v_addc_co_u32 (VOP3)", "v_cndmask_b32 (VOP3)",
               "field-product mix (6 mad, 1 cndmask, 2 subb, 3 mov, 4 add)",
               "v_add_u32_e64 (VOP3 encoding)", "v_add_co_u32_e32 (VOP2, VCC)",
               "64-bit add on VCC (add_co, 2 add, addc; VOP2)", "v_cndmask_b32_e32 (VOP2, VCC)", "v_mov_b32 (VOP1)",
               "v_mov_b64 (VOP1)", "v_lshl_add_u64 (VOP3)", "v_add_u32 + literal", "v_add_u32 / s_nop 0",
               "v_xor_b32 (VOP2)", "v_add3_u32 (VOP3)", "v_lshlrev_b32 (VOP2)",
               "64-bit sub on VCC (sub_co, s_nop 1, subb; VOP2)"]


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-fuse", action="store_true",
                    help="commit with separate zkie_lde_batch and zkie_merkle_commit calls (the leaf "
                         "kernel re-reads the codeword) instead of zkie_lde_commit")
    ap.add_argument("--cpu-rows", type=int, default=1 << 23,
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
    ap.add_argument("--valu-peak", action="store_true",
                    help="only run the VALU issue-rate probe (every kind) and print its JSON")
    ap.add_argument("--copy-ceiling", action="store_true",
                    help="only time plain device-to-device copies and fills of 8 GiB (the practical "
                         "HBM ceiling of a streaming kernel) and print their JSON")
    ap.add_argument("--probe-ms", type=float, default=60.0,
                    help="approximate duration of each probe launch")
    ap.add_argument("--ingest-counters", metavar="DIR",
                    help="read rocprofv3 --pmc CSVs under DIR (subfolders fetch, write, valu) of a "
                         "'bench.py --steps 1 --warmup 1 --no-cpu-baseline --copy-calibration 1024' "
                         "run and write profiles/commit_step_counters.json")
    return ap.parse_args()


# ---------------------------------------------------------------------------
# Kernel sources and the counter profile measured on them.

# Translation units whose kernels the step launches (every header counts).
STEP_SOURCES = ("runtime.hip", "ntt.hip", "merkle.hip", "fold.hip")


def source_hash() -> str:
    """Hash of the step's kernel sources: a counter profile is valid only for
    the code it was measured on."""
    h = hashlib.sha256()
    for path in sorted(glob.glob(os.path.join(ROOT, "zkie_amd", "csrc", "*"))):
        if path.endswith(".hpp") or os.path.basename(path) in STEP_SOURCES:
            h.update(os.path.basename(path).encode())
            with open(path, "rb") as f:
                h.update(f.read())
    return h.hexdigest()[:16]


def load_counters():
    """The committed per-launch counters, or (None, reason) when missing or
    measured on other kernel sources."""
    if not os.path.exists(COUNTERS_JSON):
        return None, "no counter profile"
    with open(COUNTERS_JSON) as f:
        prof = json.load(f)
    if prof.get("source_hash") != source_hash():
        return None, (f"counter profile measured on sources {prof.get('source_hash')}, "
                      f"kernels now {source_hash()}: stale, not used")
    return prof, None


# ---------------------------------------------------------------------------
# VALU issue-rate probe.

def probe_lib():
    import ctypes

    path = os.path.join(ROOT, "zkie_amd", "libzkie_valu_probe.so")
    if not os.path.exists(path):
        raise ImportError(f"{path} is missing: build with python -m zkie_amd.build")
    L = ctypes.CDLL(path)
    L.zkie_valu_probe_run.argtypes = [ctypes.c_int, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p,
                                      ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_uint64)]
    L.zkie_valu_probe_run.restype = ctypes.c_int
    return L


def valu_probe(kinds, target_ms: float = 60.0):
    """Issue rate of each probe kind: 8192 workgroups of 256 threads (8 waves
    per SIMD on every CU, four times over), iterations scaled so a launch
    takes about target_ms; the best of three launches."""
    import ctypes

    from zkie_amd import _native as N

    L = probe_lib()
    blocks = 8192
    out = N.DeviceBuffer(blocks * 256 // 2)
    res = {}
    for kind in kinds:
        ms, wi = ctypes.c_double(), ctypes.c_uint64()
        iters = 256
        N.check(L.zkie_valu_probe_run(kind, blocks, iters, out.addr, ctypes.byref(ms), ctypes.byref(wi)),
                "valu probe")
        iters = min(1 << 22, max(256, int(iters * target_ms / max(ms.value, 1e-3))))
        best = None
        for _ in range(3):
            N.check(L.zkie_valu_probe_run(kind, blocks, iters, out.addr, ctypes.byref(ms), ctypes.byref(wi)),
                    "valu probe")
            rate = wi.value / (ms.value * 1e-3)
            if best is None or rate > best[0]:
                best = (rate, ms.value, wi.value)
        rate, t, w = best
        res[kind] = {"kind": PROBE_KINDS[kind], "wave_instr": w, "ms": round(t, 3),
                     "wave_instr_per_s": rate, "per_cu_per_clock": rate / CUS / CLOCK_HZ}
    return res


# ---------------------------------------------------------------------------
# CPU baseline.

def copy_ceiling(gib: int = 8, reps: int = 5):
    """HBM rate of the runtime's own device-to-device copy (reads and writes
    `gib` GiB) and fill (writes `gib` GiB), the practical ceilings of a
    streaming kernel with a 1:1 and a write-only mix; host clock around
    `reps` synchronous repetitions after one untimed."""
    from zkie_amd import _native as N
    from zkie_amd._native import DeviceBuffer
    L = N.load()
    nbytes = gib << 30
    src, dst = DeviceBuffer(nbytes // 8), DeviceBuffer(nbytes // 8)
    res = {}
    for name, fn, moved in (("copy", lambda: L.zkie_memcpy_dtod(dst.addr, src.addr, nbytes, None), 2 * nbytes),
                            ("fill", lambda: L.zkie_memset(dst.addr, 0, nbytes), nbytes)):
        N.check(fn(), name)
        N.check(L.zkie_device_synchronize(), "sync")
        t0 = time.perf_counter()
        for _ in range(reps):
            N.check(fn(), name)
        N.check(L.zkie_device_synchronize(), "sync")
        dt = (time.perf_counter() - t0) / reps
        res[name] = {"bytes": moved, "ms": dt * 1e3, "GB_per_s": moved / dt / 1e9,
                     "frac_of_8TBps": moved / dt / 8e12}
    return res


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(wl, rows: int, threads: int = 0):
    """The CPU baseline (oracle/cpu_baseline.c: the reference CPU commit path
    restated with AVX2-packed Goldilocks arithmetic and OpenMP, bit-identical
    to the oracle) on a bounded sample of the same workload, on `threads`
    host threads (0: the process's CPU share, OMP_NUM_THREADS when set, else
    every core the OS shows)."""
    from oracle import cpu_baseline as CB
    from oracle import oracle as O
    from zkie_amd import configs as C

    nproc = os.cpu_count() or 1
    threads = threads or min(int(os.environ.get("OMP_NUM_THREADS") or nproc), nproc)
    CB.set_threads(threads)
    CB.set_constants(*O.p2_constants())
    sample = wl.scaled(rows)
    data = O.gen_uniform(C.SEED_DATA, sample.elems).reshape(sample.rows, sample.cols)
    ch = C.challenges(wl.fold_k) if wl.fold_k else None
    t0 = time.perf_counter()
    cw = CB.lde_batch(data, sample.log_blowup)
    _, root = CB.merkle_commit(cw)
    if ch is not None:
        CB.fold_rows(cw, wl.fold_k, ch)
    dt = time.perf_counter() - t0
    return {
        "value": sample.elems / dt,
        "unit": "elem/s",
        "cores": threads,
        "nproc": nproc,
        "kind": "port",
        "isa": "AVX2 (4 x u64 lanes), OpenMP",
        "cpu": cpu_model(),
        "sample": f"{sample.rows} rows x {sample.cols} cols, blowup {1 << sample.log_blowup}, "
                  f"LDE + Merkle root + fold k={wl.fold_k}; {dt:.2f} s wall",
    }


# ---------------------------------------------------------------------------
# Extra measurements.

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
    bytes: both tables read once (f: 8 B per base entry, h: 16 B) and the two
    folded EF tables of 2^(t - k) entries written. The library runs the
    rounds in passes (two rounds per pass on tables of 2^20 entries or more,
    up to four otherwise); pass_bytes is what those passes move."""
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
    kern = {name: N.profile_query(name) for name in ("sumcheck_pass", "sumcheck_finish")}
    N.profile_enable(False)
    alg = (1 << t) * (8 + 16) + (1 << (t - k)) * 32
    pass_bytes, i = 0, 0
    while i < k:
        m = t - i
        kk = min(2 if m >= 20 else 4, k - i)
        pass_bytes += (1 << m) * ((8 if i == 0 else 16) + 16) + (1 << (m - kk)) * 32
        i += kk
    dev_ms = sum(ms for _, ms in kern.values()) / reps
    return {"table": f"2^{t} base x EF weights", "rounds": k, "ms_per_call": round(dt * 1e3, 3),
            "kernel_ms_per_call": round(dev_ms, 3), "alg_bytes": alg, "pass_bytes": pass_bytes,
            "GB_per_s_kernels": round(pass_bytes / (dev_ms * 1e-3) / 1e9, 1) if dev_ms else None,
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


# ---------------------------------------------------------------------------
# Rooflines.

def alg_bytes(wl, lens):
    """Algorithmic HBM bytes of each stage: the LDE reads the input and
    writes the codeword; the Merkle tree writes every digest once (the
    codeword read is shared with the LDE's write in the fused minimum); the
    fold reads the codeword and writes one EF element per row."""
    n, w = wl.codeword_rows, wl.cols
    out = {"lde": wl.elems * 8 + n * w * 8, "merkle": sum(lens) * 64}
    out["lde+merkle"] = out["lde"] + out["merkle"]
    if wl.fold_k:
        out["fold"] = n * w * 8 + n * 16
    return out


def roofline(t_s: float, nbytes: float, valu_instr, valu_peak: float, traffic=None):
    """Both bounds of a kernel or stage taking t_s seconds."""
    hbm = {"achieved": nbytes / t_s / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
           "frac": nbytes / t_s / 1e9 / HBM_PEAK_GBS, "alg_bytes": nbytes, "traffic": traffic,
           "t_bound_ms": nbytes / (HBM_PEAK_GBS * 1e9) * 1e3}
    r = {"hbm": hbm, "valu": None, "bound": "hbm", "t_bound_ms": hbm["t_bound_ms"], "ms": t_s * 1e3,
         "frac": hbm["frac"]}
    if valu_instr:
        v = {"achieved": valu_instr / t_s, "peak": valu_peak, "unit": "wave-instr/s",
             "frac": valu_instr / t_s / valu_peak, "wave_instr": valu_instr,
             "t_bound_ms": valu_instr / valu_peak * 1e3}
        r["valu"] = v
        if v["t_bound_ms"] > hbm["t_bound_ms"]:
            r.update(bound="valu", t_bound_ms=v["t_bound_ms"], frac=v["frac"])
    return r


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for {args.gpus}); the multi-GPU "
              "sharding of this path is a design, not a measured configuration.", file=sys.stderr)
        sys.exit(2)
    if args.ingest_counters:
        ingest_counters(args.ingest_counters)
        return
    if args.valu_peak:
        res = valu_probe(range(len(PROBE_KINDS)), args.probe_ms)
        print(json.dumps({"valu_issue_rates": list(res.values()), "cus": CUS, "clock_hz": CLOCK_HZ}), flush=True)
        return
    if args.copy_ceiling:
        print(json.dumps({"copy_ceiling": copy_ceiling()}), flush=True)
        return

    from zkie_amd import _native as N
    from zkie_amd import configs as C
    from zkie_amd.pcs import fold_rows_device
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
    L = N.load()
    import numpy as np
    root = np.zeros(8, np.uint64)
    stream = N.Stream()

    def step():
        # encode then commit (zkie_lde_commit: the last NTT pass of 16-wide
        # rows hashes the rows it produces)
        if args.no_fuse:
            N.check(L.zkie_lde_batch(d_in.addr, wl.rows, w, wl.log_blowup, 1, d_cw.addr, stream.handle), "lde")
            N.check(L.zkie_merkle_commit(d_cw.addr, n, w, d_layers.addr, N.p(root), stream.handle), "commit")
        else:
            N.check(L.zkie_lde_commit(d_in.addr, wl.rows, w, wl.log_blowup, 1, d_cw.addr, d_layers.addr,
                                      N.p(root), stream.handle), "zkie_lde_commit")
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

    # Issue peak of the VALU, measured now: the fastest of the plain 32-bit
    # operations (v_add_u32 in both encodings, v_mov_b32) and, for reference,
    # the mix of the field product the Poseidon2 kernels run.
    probe = valu_probe([0, 7, 11, 6], args.probe_ms)
    valu_peak = max(p["wave_instr_per_s"] for p in probe.values())

    counters, stale = load_counters() if args.config == 3 else (None, "counters are profiled at configuration 3")
    kc = (counters or {}).get("kernels", {})

    def per_step(name, field):
        """A kernel's counter summed over one step (None without a valid profile)."""
        return kc.get(name, {}).get(field + "_per_step")

    ab = alg_bytes(wl, lens)
    step_ms = {k: ms / args.steps for k, (cnt, ms) in per_kernel.items()}
    # Dominant kernel: the Merkle leaf hash (or the fused last NTT pass + leaf hash).
    dom = "ntt_last_leaf" if "ntt_last_leaf" in per_kernel else "p2_leaf"
    dn, dms = per_kernel.get(dom, (0, 0.0))
    dom_avg_s = dms / max(dn, 1) * 1e-3
    # Its algorithmic bytes per launch: read the rows (or, fused, the last
    # pass's input) and write the layer-0 digests (and, fused, the codeword).
    dom_bytes = n * w * 8 + n * 64 + (n * w * 8 if dom == "ntt_last_leaf" else 0)
    dom_launches = dn / args.steps
    dom_traffic = dom_valu = None
    if per_step(dom, "fetch_bytes") is not None:
        dom_traffic = (per_step(dom, "fetch_bytes") + per_step(dom, "write_bytes")) / dom_launches
        dom_valu = per_step(dom, "valu_wave_instr") / dom_launches
    dom_roof = roofline(dom_avg_s, dom_bytes, dom_valu, valu_peak, dom_traffic)

    stages = {}
    fused = "ntt_last_leaf" in per_kernel
    for st, names in STAGE_KERNELS.items():
        if st not in ab or (fused and st in ("lde", "merkle")) or (not fused and st == "lde+merkle"):
            continue
        ms = sum(step_ms.get(k, 0.0) for k in names)
        if not ms:
            continue
        vi = tr = None
        if counters:
            vi = sum(per_step(k, "valu_wave_instr") or 0 for k in names if k in per_kernel)
            tr = sum((per_step(k, "fetch_bytes") or 0) + (per_step(k, "write_bytes") or 0)
                     for k in names if k in per_kernel)
        stages[st] = roofline(ms * 1e-3, ab[st], vi, valu_peak, tr)
    step_bytes = ab["lde+merkle"] + ab.get("fold", 0)
    step_valu = sum(s["valu"]["wave_instr"] for s in stages.values() if s["valu"]) if counters else None
    step_roof = roofline(t, step_bytes, step_valu, valu_peak)

    def headline(r, kernel):
        """The contract's roofline object for the binding component."""
        c = r[r["bound"]]
        return {"bound": r["bound"], "kernel": kernel, "achieved": c["achieved"], "peak": c["peak"],
                "unit": c["unit"], "frac": c["frac"], "traffic": r["hbm"]["traffic"],
                "avg_ms": r["ms"], "hbm": r["hbm"], "valu": r["valu"]}

    out = {
        "metric": METRIC,
        "value": wl.elems / t,
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
        "roofline": headline(dom_roof, dom),
        "step_roofline": headline(step_roof, "step"),
        "step_hbm_frac": step_roof["hbm"]["frac"],
        "stages": stages,
        "stage_ms_per_step": {k: round(v, 3) for k, v in step_ms.items()},
        "valu_peak": {"wave_instr_per_s": valu_peak, "probe": list(probe.values()),
                      "source": "libzkie_valu_probe.so, measured in this run"},
        "counters": {"source": os.path.relpath(COUNTERS_JSON, ROOT), "used": counters is not None,
                     "note": stale, "source_hash": source_hash()},
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


# ---------------------------------------------------------------------------
# Counter ingestion (rocprofv3 --pmc CSV -> profiles/commit_step_counters.json).

# rocprofv3 kernel names -> the library's profiler names.
KERNEL_NAMES = [("ntt_last_leaf_kernel", "ntt_last_leaf"), ("leaf_kernel", "p2_leaf"),
                ("compress_x16_kernel", "p2_compress"), ("compress_kernel", "p2_compress"),
                ("subtree_kernel", "p2_subtree"), ("fold_kernel", "fold_rows")]
COPY_KERNEL = "copyBuffer"


def _kernel_key(name: str, grid: int, first_grids: dict):
    for pat, key in KERNEL_NAMES:
        if pat in name:
            return key
    if "ntt_pass_kernel" in name:
        # named by launch order afterwards (first, middle, last pass of a step)
        return name
    return None


def ingest_counters(d: str):
    """Per-launch counters of the step's kernels from three rocprofv3 runs
    (one counter group each) of one step: FETCH_SIZE and WRITE_SIZE (KiB,
    scaled by what they read for the 0.5 GiB dispatches of the trailing
    device-to-device copies) and SQ_INSTS_VALU (wave-instructions)."""
    vals = {}  # (group, dispatch) -> (kernel, grid, value)
    for group, counter in (("fetch", "FETCH_SIZE"), ("write", "WRITE_SIZE"), ("valu", "SQ_INSTS_VALU")):
        files = glob.glob(os.path.join(d, group, "**", "*counter_collection.csv"), recursive=True)
        if not files:
            raise SystemExit(f"no counter_collection.csv under {os.path.join(d, group)}")
        rows = {}
        with open(files[0]) as f:
            for r in csv.DictReader(f):
                if r.get("Counter_Name") != counter:
                    continue
                disp = int(r["Dispatch_Id"])
                rows.setdefault(disp, [r["Kernel_Name"], int(r.get("Grid_Size", 0) or 0), 0.0])
                rows[disp][2] += float(r["Counter_Value"])
        vals[group] = rows
    # Calibration from the trailing device-to-device copies: one dispatch of
    # 1 GiB each (the largest copy dispatches of the run; smaller ones are
    # the run's own small copies).
    copy_bytes = 1 << 30

    def scale(group):
        c = [v for v in vals[group].values() if COPY_KERNEL in v[0]]
        if not c:
            raise SystemExit(f"no copy dispatch in the {group} run (run with --copy-calibration 1024)")
        big = max(x[1] for x in c)
        kib = sorted(x[2] for x in c if x[1] == big)[len([x for x in c if x[1] == big]) // 2]
        return copy_bytes / kib

    fs, ws_ = scale("fetch"), scale("write")
    steps_profiled = 2  # --warmup 1 --steps 1
    kernels = {}
    ntt_order = []
    for group, field, sc in (("fetch", "fetch_bytes", fs), ("write", "write_bytes", ws_),
                             ("valu", "valu_wave_instr", 1.0)):
        per = {}
        for disp in sorted(vals[group]):
            name, grid, v = vals[group][disp]
            key = _kernel_key(name, grid, {})
            if key is None:
                continue
            if "ntt_pass_kernel" in key and key not in ntt_order:
                ntt_order.append(key)
            per.setdefault(key, []).append(v * sc)
        for key, vs in per.items():
            kernels.setdefault(key, {})[field + "_per_step"] = sum(vs) / steps_profiled
            kernels[key]["launches_per_step"] = len(vs) / steps_profiled
    # Name the NTT passes by their order in the step, as the library's timers
    # do (with the last pass fused with the leaf hash, no plain last pass).
    names = {}
    fused = "ntt_last_leaf" in kernels
    for i, k in enumerate(ntt_order):
        last = i == len(ntt_order) - 1 and not fused
        names[k] = "ntt_pass_first" if i == 0 else ("ntt_pass_last" if last else "ntt_pass_mid")
    out = {}
    for k, v in kernels.items():
        out[names.get(k, k)] = dict(v, rocprof_name=k)
    prof = {"source_hash": source_hash(), "workload": "uniform_2^24x16_blowup4_root_fold4",
            "fetch_scale": fs, "write_scale": ws_,
            "command": "rocprofv3 --pmc {FETCH_SIZE | WRITE_SIZE | SQ_INSTS_VALU} --output-format csv "
                       "-d gpurun_out/prof/<group> -o bench -- python3 bench.py --steps 1 --warmup 1 "
                       "--no-cpu-baseline --copy-calibration 1024",
            "kernels": out}
    with open(COUNTERS_JSON, "w") as f:
        json.dump(prof, f, indent=1)
    print(json.dumps(prof, indent=1))


if __name__ == "__main__":
    main()
