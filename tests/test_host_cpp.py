"""Runs the C++20 host tests (tests/cpp/, built by python -m synapse_amd.build):
the graph builder and planner on the CPU, the session through the C ABI on
the GPU against the CPU oracle."""
from __future__ import annotations

import pathlib
import subprocess

import pytest

BIN = pathlib.Path(__file__).resolve().parent / "cpp" / "_bin"


def _run(name: str) -> None:
    exe = BIN / name
    if not exe.exists():
        pytest.fail(f"{exe} is missing: build with `python -m synapse_amd.build`")
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout + proc.stderr


def test_graph_builder_and_planner():
    _run("test_graph")


@pytest.mark.gpu
def test_session_against_the_oracle():
    _run("test_session")
