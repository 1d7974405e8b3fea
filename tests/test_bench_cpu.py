"""CPU checks of bench.py: every name a function reads is defined (the
benchmark itself only runs on a GPU), the multi-GPU request exits with its
message before touching a device, and the profile summaries the bench reads
traffic from exist and carry a traffic line."""
import builtins
import os
import subprocess
import symtable
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def _free_globals(table, out):
    """Names that function scopes read as module globals."""
    for child in table.get_children():
        if child.get_type() == "function":
            for sym in child.get_symbols():
                if sym.is_referenced() and sym.is_global() and not sym.is_declared_global():
                    out.add((child.get_name(), sym.get_name()))
        _free_globals(child, out)


def test_bench_functions_read_defined_names():
    src = open(BENCH).read()
    top = symtable.symtable(src, BENCH, "exec")
    defined = {s.get_name() for s in top.get_symbols() if s.is_assigned() or s.is_imported()}
    defined |= set(dir(builtins))
    used = set()
    _free_globals(top, used)
    missing = sorted((fn, name) for fn, name in used if name not in defined)
    assert not missing, missing


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, BENCH, "--gpus", "2"], capture_output=True, text=True,
                       timeout=120, cwd=ROOT)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr) or "1 GPU" in (r.stdout + r.stderr)


def test_bench_traffic_profiles_exist():
    sys.path.insert(0, ROOT)
    try:
        import importlib
        bench = importlib.import_module("bench")
    finally:
        sys.path.pop(0)
    for key, name in bench.PROFILES.items():
        path = os.path.join(ROOT, "profiles", name)
        assert os.path.exists(path), (key, name)
    for key in ("c2", "c2_b2", "c2bwd"):
        assert bench.measured_traffic(key) is not None, key
