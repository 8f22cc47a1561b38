"""bench.py's names resolve: every name a function of bench.py reads as a global is defined at module level or is a
builtin (a static check on the CPU; the benchmark itself needs the GPU)."""
import builtins
import pathlib
import symtable

ROOT = pathlib.Path(__file__).resolve().parents[1]


def _unresolved(path):
    src = path.read_text()
    top = symtable.symtable(src, str(path), "exec")
    defined = {s.get_name() for s in top.get_symbols() if s.is_assigned() or s.is_imported()}
    defined |= set(dir(builtins))
    bad = []

    def walk(t, where):
        for ch in t.get_children():
            name = f"{where}.{ch.get_name()}"
            for s in ch.get_symbols():
                if s.is_global() and s.is_referenced() and s.get_name() not in defined:
                    bad.append(f"{name}: {s.get_name()}")
            walk(ch, name)

    walk(top, path.name)
    return bad


def test_bench_globals_resolve():
    assert _unresolved(ROOT / "bench.py") == []


def test_graft_entry_globals_resolve():
    assert _unresolved(ROOT / "__graft_entry__.py") == []
