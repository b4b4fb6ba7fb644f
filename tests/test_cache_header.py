"""The batch cache header of the C++ host interface (zkie::write_header /
read_header over crates/zkie-core/src/pcs/cache.rs:7-70) on the CPU:
tests/cpp/test_cache_header.cpp, built with g++ alone, checks the bytes of
the reference's own cache fixture (whir.rs:875-886) laid out in bincode
1.3.3's encoding, the round trip and the refusals. The layout of bincode's
integers, strings and sequences is pinned by its specification; that p3's
MerkleCap and Goldilocks serialise as a sequence of digests of u64 (the
commitment part) is restated, parity unpinned."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def test_cache_header(tmp_path):
    exe = tmp_path / "test_cache_header"
    r = subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-I" + os.path.join(ROOT, "include"),
                        os.path.join(HERE, "cpp", "test_cache_header.cpp"), "-o", str(exe)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and "ALL PASS" in r.stdout, r.stdout + r.stderr
