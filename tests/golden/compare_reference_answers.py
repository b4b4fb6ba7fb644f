"""Compare the output of the reference-side program of INTEGRATION.md
(crates/zkie-core/examples/p2_known_answers.rs, run where p3 0.7.0 and rand
0.10 are available) with this repository's frozen restatement:
tests/golden/known_answers.json, the internal diagonal restated from
poseidon2_merkle.cu:111-142, W = 7 and TWO_ADIC_GENERATORS[k] =
7^((p-1)/2^k).

  python3 tests/golden/compare_reference_answers.py answers.json

Prints one line per compared field and exits non-zero on any difference."""
import json
import os
import sys

P = 0xFFFFFFFF00000001
HERE = os.path.dirname(os.path.abspath(__file__))


def restated():
    inv = lambda x: pow(x, P - 2, P)  # noqa: E731
    i2, i8, i16, i32 = inv(2), inv(8), inv(16), inv(32)
    diag = [P - 2, 1, 2, i2, 3, 4, P - i2, P - 3, P - 4, i8, i16, i32, P - i8, P - i16, P - i32, inv(1 << 32)]
    ka = json.load(open(os.path.join(HERE, "known_answers.json")))
    return {
        "p2_constants": ka["p2_constants"],
        "matrix_diag_16": [f"{x:016x}" for x in diag],
        "ext_w": f"{7:016x}",
        "two_adic_generators": [f"{pow(7, (P - 1) >> k, P):016x}" for k in range(33)],
        "p2_permute_iota": ka["p2_permute"]["iota"]["out"],
        "leaf_hash_9": ka["leaf_hash"]["9"]["digest"],
        "compress": ka["compress"]["out"],
    }


def compare(got) -> int:
    """Print one line per field of the restatement; return the number of
    fields that differ or are missing."""
    want = restated()
    bad = 0
    for key, exp in want.items():
        if key not in got:
            print(f"{key}: missing")
            bad += 1
            continue
        ok = got[key] == exp
        bad += not ok
        print(f"{key}: {'same' if ok else 'DIFFERENT'}")
    return bad


def main(path):
    sys.exit(1 if compare(json.load(open(path))) else 0)


if __name__ == "__main__":
    main(sys.argv[1])
