"""The Node host (gemma-webgpu-engine_amd/node, the N-API addon over the C ABI)
on a machine without a GPU: the addon loads and exports every entry point,
the option surface returns the reference's known answers, SeededRandom agrees
with the oracle, and compute calls fail loudly without a device."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def run_node_tests(script, timeout):
    node = shutil.which("node")
    if node is None:
        pytest.skip("node is not installed")
    proc = subprocess.run([node, os.path.join(ROOT, "tests", "node", script)], cwd=ROOT, capture_output=True,
                          text=True, timeout=timeout)
    print(proc.stdout)
    print(proc.stderr)
    assert proc.returncode == 0, proc.stdout[-4000:] + proc.stderr[-4000:]
    assert "FAIL" not in proc.stdout
    return proc.stdout


def test_node_host_surface_without_gpu():
    addon = os.path.join(ROOT, "gemma-webgpu-engine_amd", "lib", "gsample_node.node")
    if not os.path.exists(addon):
        pytest.fail("gsample_node.node is not built; run __graft_entry__.build()")
    out = run_node_tests("cpu_surface.js", 120)
    assert "all 9 passed" in out


def test_constraint_compiler_without_gpu():
    """Regex / JSON / JSON Schema constraints compiled to byte-level DFA
    tables: the reference's constraint known answers, RegExp full-match
    acceptance, and the reference's pending UTF-8 byte walk."""
    out = run_node_tests("constraint_compiler.js", 300)
    assert "all 14 passed" in out
