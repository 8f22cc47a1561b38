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


def test_pmc_kernel_and_scale():
    """The live traffic figure's parsing: a counter spread over rows of one dispatch adds up, the scale comes from the
    last copies only (the arena's earlier copies are of other sizes), and too few dispatches give None."""
    import bench
    rows = []
    for d in range(3):   # an arena copy first: not among the last 4
        rows.append(dict(Dispatch_Id=str(d), Kernel_Name="__amd_rocclr_copyBuffer", Counter_Name="FETCH_SIZE",
                         Counter_Value="999999"))
    for d in range(3, 3 + 64):
        for part in (100.0, 25.0):   # two rows of one dispatch
            rows.append(dict(Dispatch_Id=str(d), Kernel_Name="xs::moe_decode_t1_kernel<12, 14, 2>",
                             Counter_Name="FETCH_SIZE", Counter_Value=str(part)))
        rows.append(dict(Dispatch_Id=str(d), Kernel_Name="xs::moe_decode_t1_kernel<12, 14, 2>",
                         Counter_Name="WRITE_SIZE", Counter_Value="7"))
    for d in range(67, 71):
        rows.append(dict(Dispatch_Id=str(d), Kernel_Name="__amd_rocclr_copyBuffer", Counter_Name="FETCH_SIZE",
                         Counter_Value="131072"))
    mean, scale, n = bench.pmc_kernel_and_scale(rows, "FETCH_SIZE", "moe_decode_t1_kernel", 262144.0)
    assert (mean, scale, n) == (125.0, 2.0, 64)
    assert bench.pmc_kernel_and_scale(rows[:50], "FETCH_SIZE", "moe_decode_t1_kernel", 262144.0) is None
    # a small copy after the calibration (a status read) makes the last 4 differ: refused, not averaged in
    tail = rows + [dict(Dispatch_Id="71", Kernel_Name="__amd_rocclr_copyBuffer", Counter_Name="FETCH_SIZE",
                        Counter_Value="1")]
    assert bench.pmc_kernel_and_scale(tail, "FETCH_SIZE", "moe_decode_t1_kernel", 262144.0) is None
