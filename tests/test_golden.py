"""Golden fixtures (tests/golden/, written by tests/golden/make_golden.py).

CPU: the oracle reproduces the fixtures (the PRNG vectors are published
reference outputs; the rest freeze the oracle). GPU: libzkie_hip.so
reproduces them, including the full-size roots and checksums of all five
workloads."""
import json
import os

import numpy as np
import pytest

from zkie_amd import configs as C

HERE = os.path.dirname(os.path.abspath(__file__))
KA = json.load(open(os.path.join(HERE, "golden", "known_answers.json")))
WL_PATH = os.path.join(HERE, "golden", "workloads.json")
WL = json.load(open(WL_PATH)) if os.path.exists(WL_PATH) else {}


def u(hexlist):
    return np.array([int(x, 16) for x in hexlist], np.uint64)


def test_published_prng_vectors(oracle):
    r = oracle.Xoshiro256pp(state=[1, 2, 3, 4])
    assert [r.next_u64() for _ in range(10)] == KA["xoshiro256pp_state_1_2_3_4"]
    assert [f"{x:016x}" for x in oracle.splitmix64(0, 3)] == KA["splitmix64_seed_0"]


def test_oracle_reproduces_fixtures(oracle):
    a, b, c, d = oracle.p2_constants()
    k = KA["p2_constants"]
    assert (a == u(k["rc_init"])).all() and (b == u(k["rc_final"])).all()
    assert (c == u(k["rc_internal"])).all() and d == int(k["diag15"], 16)
    for v in KA["p2_permute"].values():
        assert (oracle.p2_permute(u(v["in"])) == u(v["out"])).all()
    for v in KA["leaf_hash"].values():
        assert (oracle.leaf_hash(u(v["row"])) == u(v["digest"])).all()
    cp = KA["compress"]
    assert (oracle.compress(u(cp["left"]), u(cp["right"])) == u(cp["out"])).all()
    for key, v in KA["dft"].items():
        lg, w = map(int, key.split("x"))
        assert (oracle.dft_batch(u(v["in"]).reshape(1 << lg, w)).reshape(-1) == u(v["out"])).all()
    f = KA["fold_k4"]
    assert (oracle.fold_rows(u(f["rows"]).reshape(4, 16), 4, u(f["r"]).reshape(4, 2), False)
            .reshape(-1) == u(f["out"])).all()


def test_workload_fixtures_cover_all_configs():
    assert sorted(WL) == [str(n) for n in sorted(C.CONFIGS)], "run make_golden.py --full"


@pytest.mark.gpu
def test_gpu_reproduces_known_answers(native):
    from zkie_amd import pcs

    print("CASE golden known answers", flush=True)
    g = native.p2_default_constants()
    k = KA["p2_constants"]
    assert (g[0] == u(k["rc_init"])).all() and (g[1] == u(k["rc_final"])).all()
    assert (g[2] == u(k["rc_internal"])).all() and g[3] == int(k["diag15"], 16)
    mmcs = pcs.HipMerkleTreeMmcs()
    for w, v in KA["leaf_hash"].items():
        root, _ = mmcs.commit(u(v["row"]).reshape(1, int(w)))  # one row: root = leaf digest
        assert (root == u(v["digest"])).all()
    for key, v in KA["dft"].items():
        lg, w = map(int, key.split("x"))
        got = pcs.HipDft().dft_batch(u(v["in"]).reshape(1 << lg, w))
        assert (got.reshape(-1) == u(v["out"])).all()
    f = KA["fold_k4"]
    got = pcs.fold_rows(u(f["rows"]).reshape(4, 16), 4, u(f["r"]).reshape(4, 2), False)
    assert (got.reshape(-1) == u(f["out"])).all()


@pytest.mark.gpu
@pytest.mark.parametrize("number", sorted(C.CONFIGS))
def test_gpu_full_size_workload_matches_fixture(native, oracle, number):
    from zkie_amd import pipeline as PL
    from zkie_amd._native import DeviceBuffer

    if str(number) not in WL:
        pytest.skip("fixture not generated")
    ref = WL[str(number)]
    wl = C.CONFIGS[number]
    print("CASE golden workload", wl.name, flush=True)
    data = PL.workload_inputs(wl)
    assert f"{oracle.checksum(data):016x}" == ref["input_checksum"]
    out = PL.run_workload(wl, DeviceBuffer.from_array(data), with_openings=bool(wl.queries))
    del data
    assert len(out.rounds) == len(ref["rounds"])
    for rnd, r in zip(out.rounds, ref["rounds"]):
        assert rnd.rows == r["rows"] and rnd.width == r["width"]
        assert (rnd.tree.root == u(r["root"])).all(), "root differs from the oracle's"
        if "queries" in r:
            assert [int(i) for i in rnd.queries] == r["queries"]
            assert (rnd.opened_rows[0] == u(r["first_row"])).all()
            assert (rnd.paths[0].reshape(-1) == u(r["first_path"])).all()
            assert rnd.pruned.shape[0] == r["pruned_count"]
        if rnd.rows * rnd.width <= (1 << 27):
            assert f"{oracle.checksum(rnd.codeword.download()):016x}" == r["codeword_checksum"]
    if "fold_checksum" in ref:
        assert f"{oracle.checksum(out.fold.download()):016x}" == ref["fold_checksum"]
    for (buf, _), cs in zip(out.tables, ref.get("table_checksums", [])):
        assert f"{oracle.checksum(buf.download()):016x}" == cs


def test_reference_comparison_script_matches_the_oracle(oracle):
    """tests/golden/compare_reference_answers.py (the check a holder of the
    external crates runs) states the same constants as the oracle."""
    import importlib.util

    spec = importlib.util.spec_from_file_location("cra", os.path.join(HERE, "golden", "compare_reference_answers.py"))
    cra = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(cra)
    w = cra.restated()
    a, b, c, d = oracle.p2_constants()
    assert w["p2_constants"]["rc_init"] == [f"{int(x):016x}" for x in a]
    assert int(w["matrix_diag_16"][15], 16) == d
    assert [int(x, 16) for x in w["two_adic_generators"]] == [oracle.two_adic_generator(k) for k in range(33)]
    iota = np.arange(16, dtype=np.uint64)
    assert [int(x, 16) for x in w["p2_permute_iota"]] == [int(x) for x in oracle.p2_permute(iota)]
    # the restatement compares equal to itself, and a single planted
    # difference (one diagonal word) or a missing field is reported
    assert cra.compare(w) == 0
    planted = dict(w, matrix_diag_16=list(w["matrix_diag_16"]))
    planted["matrix_diag_16"][7] = f"{(int(planted['matrix_diag_16'][7], 16) + 1) % (2**64):016x}"
    assert cra.compare(planted) == 1
    assert cra.compare({k: v for k, v in w.items() if k != "ext_w"}) == 1
