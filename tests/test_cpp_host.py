"""The C++ host interface (include/zkie_hip.hpp): the header compiles on its
own (CPU), and its engines match the oracle on the GPU
(tests/cpp/test_host_mirror.cpp, built by __graft_entry__.build())."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def test_header_compiles_standalone(tmp_path):
    src = tmp_path / "inc.cpp"
    src.write_text('#include "zkie_hip.hpp"\nint main() { zkie::HipDft d; (void)d; return 0; }\n')
    r = subprocess.run(["g++", "-std=c++17", "-Wall", "-Werror", "-fsyntax-only",
                        "-I" + os.path.join(ROOT, "include"), str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


@pytest.mark.gpu
def test_cpp_host_interface_matches_oracle():
    binary = os.path.join(HERE, "cpp", "test_host_mirror")
    assert os.path.exists(binary), "run __graft_entry__.build() first"
    print("CASE C++ host interface", flush=True)
    r = subprocess.run([binary], capture_output=True, text=True, timeout=300)
    print(r.stdout[-3000:], flush=True)
    assert r.returncode == 0 and "ALL PASS" in r.stdout, r.stdout + r.stderr
