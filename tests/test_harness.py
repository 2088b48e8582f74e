"""Host-side checks of the benchmark harness (no GPU)."""
import ast
import pathlib

ROOT = pathlib.Path(__file__).resolve().parents[1]
SUITE = ROOT / "strict-topk-overlap_amd" / "stk_harness" / "suite.py"


def test_every_case_keeps_the_device_inputs_its_graphs_read():
    """A captured graph holds raw addresses; torch.cuda.graph empties the
    allocator cache at every capture, so a case whose inputs die before its
    graphs are replayed replays on memory given back to the driver.  Every
    case builder must hand its device inputs to the Case (case.keep)."""
    tree = ast.parse(SUITE.read_text())
    builders = [f for f in tree.body
                if isinstance(f, ast.FunctionDef) and f.name.startswith("case_")]
    assert len(builders) >= 5
    for f in builders:
        keeps = [n for n in ast.walk(f) if isinstance(n, ast.Assign)
                 and any(isinstance(t, ast.Attribute) and t.attr == "keep" for t in n.targets)]
        assert keeps, f"{f.name} does not set case.keep"
    cases = next(n for n in tree.body if isinstance(n, ast.Assign)
                 and any(isinstance(t, ast.Name) and t.id == "CASES" for t in n.targets))
    named = {v.id for v in cases.value.values}
    assert named == {f.name for f in builders}


def test_bench_releases_graphs_with_their_inputs():
    src = (ROOT / "bench.py").read_text()
    assert "case.release()" in src and "case.graphs = {}" not in src
