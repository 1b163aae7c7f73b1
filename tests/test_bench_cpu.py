"""CPU checks of bench.py's contract that need no GPU: the one-GPU guard, the
config-group filter, that the config sections do not rebind the helpers
they share (a section assigning to `want` or `rec` would break every later
section of the default run), the cap on captured graph calls, and that no
reference build is timed (the CPU baseline runs torch and this repo's ports)."""

import ast
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def _run(*args):
    return subprocess.run([sys.executable, BENCH, *args], capture_output=True, text=True, timeout=300)


def test_more_than_one_gpu_is_refused():
    r = _run("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_unknown_config_group_is_refused():
    r = _run("--only", "C9")
    assert r.returncode == 2
    assert "unknown config groups" in r.stderr


def test_config_sections_do_not_rebind_shared_helpers():
    tree = ast.parse(open(BENCH).read())
    fn = next(n for n in ast.walk(tree) if isinstance(n, ast.FunctionDef) and n.name == "measure_configs")
    helpers = {n.name for n in fn.body if isinstance(n, ast.FunctionDef)}
    assert {"want", "rec", "nbuf_for"} <= helpers
    stored = {n.id for n in ast.walk(fn) if isinstance(n, ast.Name) and isinstance(n.ctx, ast.Store)}
    assert not (stored & helpers), stored & helpers


def test_graph_capture_is_capped():
    import importlib.util

    spec = importlib.util.spec_from_file_location("bench_mod", BENCH)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    try:
        mod._time_graph(None, None, mod.MAX_GRAPH_CALLS + 1, None)
    except AssertionError as e:
        assert "captured calls" in str(e)
    else:
        raise AssertionError("an oversized capture was not refused")


def test_no_reference_build_is_timed():
    tree = ast.parse(open(BENCH).read())
    names = {n.attr for n in ast.walk(tree) if isinstance(n, ast.Attribute)}
    assert not {a for a in names if a.startswith("ref_")}, sorted(a for a in names if a.startswith("ref_"))
