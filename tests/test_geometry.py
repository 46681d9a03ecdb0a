"""Launch geometry against workspace capacity, on the CPU: tests/geometry_check.cpp sweeps layer
shapes and call sizes through the same host arithmetic the launchers and trk_create use
(tr-infer_amd/csrc/geometry.hpp).  A grid that addresses strips past F or a workspace piece sized
below what a dispatch writes fails here without a GPU."""
from __future__ import annotations

import os
import subprocess
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), "tr-infer_amd", "csrc")


def test_launch_geometry_sweep():
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "geometry_check")
        subprocess.run(["g++", "-O1", "-std=c++17", "-Wall", "-Werror", "-I", CSRC,
                        os.path.join(HERE, "geometry_check.cpp"), "-o", exe], check=True)
        r = subprocess.run([exe], capture_output=True, text=True)
        assert r.returncode == 0, r.stdout + r.stderr
        assert r.stdout.startswith("ok ") and int(r.stdout.split()[1]) > 100000
