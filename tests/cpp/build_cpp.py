"""Build the C++ host-interface test program (tests/cpp/test_host_mirror)
against include/zkie_hip.hpp, libzkie_hip.so and the oracle library."""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
SRC = os.path.join(HERE, "test_host_mirror.cpp")
BIN = os.path.join(HERE, "test_host_mirror")


def command() -> list:
    return ["g++", "-std=c++17", "-O2", "-Wall", "-I" + os.path.join(ROOT, "include"),
            "-I" + os.path.join(ROOT, "oracle"), SRC, "-L" + os.path.join(ROOT, "zkie_amd"), "-lzkie_hip",
            "-L" + os.path.join(ROOT, "oracle"), "-lzkie_oracle",
            "-Wl,-rpath,$ORIGIN/../../zkie_amd", "-Wl,-rpath,$ORIGIN/../../oracle", "-o", BIN]


def build() -> str:
    r = subprocess.run(command(), capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("C++ host-interface test build failed:\n" + r.stderr)
    return BIN
