"""Build step: compiles libcqhip.so for gfx950 (csrc/Makefile) and, for the
tests, the CPU oracle (oracle/Makefile)."""

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def _make(directory, force):
    jobs = str(min(16, os.cpu_count() or 4))
    cmd = ["make", "-C", directory, "-j", jobs]
    if force:
        cmd.insert(1, "-B")
    subprocess.run(cmd, check=True)


def build_library(force=True):
    _make(os.path.join(HERE, "csrc"), force)


def build_oracle(force=True):
    _make(os.path.join(ROOT, "oracle"), force)


if __name__ == "__main__":
    build_library()
    build_oracle()
