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


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU's share; asked for several GPUs it exits
    with a message before touching any device."""
    import subprocess
    import sys
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert r.returncode != 0
    assert "one GPU" in r.stderr and not r.stdout.strip()


def test_paged_api_validates_on_the_host():
    """The paged entry points reject malformed batches before any launch
    (no GPU needed): wrong Q / prediction shapes, dtypes, widths and topk."""
    import sys
    import pytest
    import torch
    sys.path.insert(0, str(ROOT / "strict-topk-overlap_amd"))
    from strict_topk import paged
    r, hkv, nb, b, d, pages = 2, 2, 5, 4, 64, 30
    kv = paged.PagedKV(torch.zeros((pages, b, d), dtype=torch.bfloat16),
                       torch.zeros((pages, b, d), dtype=torch.bfloat16),
                       torch.zeros((pages, d)), torch.zeros((pages, d)),
                       torch.zeros((r, hkv, nb), dtype=torch.int32),
                       torch.full((r,), nb, dtype=torch.int32))
    assert (kv.requests, kv.hkv, kv.width, kv.pages, kv.block, kv.dim) == (r, hkv, nb, pages, b, d)
    q = torch.zeros((r, 4, d), dtype=torch.bfloat16)
    p = torch.zeros((r, 4, 3), dtype=torch.int32)
    with pytest.raises(ValueError, match="Q\\[R,Hq,D\\]"):
        paged.speculative_step(q[:1], kv, p, 2)
    with pytest.raises(ValueError, match="divisible"):
        paged.speculative_step(torch.zeros((r, 3, d), dtype=torch.bfloat16), kv, p[:, :3], 2)
    with pytest.raises(ValueError, match="P\\[R,Hq,SP\\]"):
        paged.speculative_step(q, kv, p[:, :2], 2)
    with pytest.raises(ValueError, match="int32"):
        paged.speculative_step(q, kv, p.long(), 2)
    with pytest.raises(ValueError, match="dtype"):
        paged.exact(q.half(), kv, 2)
    with pytest.raises(ValueError, match="topk"):
        paged.exact(q, kv, 0)
    with pytest.raises(ValueError, match="topk"):
        paged.exact(q, kv, 300)
    with pytest.raises(ValueError):
        paged.speculative_signed_step(q, kv, p, 2, mode="compact")
    with pytest.raises(ValueError):
        paged.speculative_signed_step(q, kv, p, 2, mass_threshold=2.0)
    with pytest.raises(TypeError):
        paged.exact(q, (kv.k_pages, kv.v_pages), 2)
    kn = torch.zeros((r, hkv, d), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="K_NEW"):
        paged.append(kv, kn[:, :1], kn, torch.zeros((r,), dtype=torch.int32))
    with pytest.raises(ValueError, match="positions"):
        paged.append(kv, kn, kn, torch.zeros((r,), dtype=torch.int64))
    with pytest.raises(ValueError, match="CUDA"):
        paged.speculative_step(q, kv, p, 2)   # a well-formed batch, but on the CPU
    with pytest.raises(ValueError, match="CUDA"):
        paged.append(kv, kn, kn, torch.zeros((r,), dtype=torch.int32))
    with pytest.raises(ValueError, match="narrower"):
        paged.pack([(torch.zeros((hkv, 6, b, d)), torch.zeros((hkv, 6, b, d)))], width=3)


def test_masks_and_token_counts_validate_on_the_host():
    """Masks and token counts are checked before any launch: a mask that is
    not on the CUDA device, a token count that does not end inside the last
    block, an ntokens tensor of the wrong dtype."""
    import sys
    import pytest
    import torch
    sys.path.insert(0, str(ROOT / "strict-topk-overlap_amd"))
    from strict_topk import kernels, paged
    st = kernels.PartialState(torch.zeros((2, 3)), torch.zeros((2, 3)), torch.zeros((2, 3, 8)))
    with pytest.raises(ValueError, match="include"):
        kernels.merge_partials(st, include=torch.ones((2, 3), dtype=torch.bool))
    k = torch.zeros((2, 3, 4, 8))
    with pytest.raises(ValueError, match="tokens"):
        paged.pack([(k, k)], tokens=[8])        # 3 blocks of 4: tokens must be in (8, 12]
    with pytest.raises(ValueError, match="tokens"):
        paged.pack([(k, k)], tokens=[13])
    r, hkv, nb, b, d, pages = 2, 2, 5, 4, 64, 30
    kv = paged.PagedKV(torch.zeros((pages, b, d), dtype=torch.bfloat16),
                       torch.zeros((pages, b, d), dtype=torch.bfloat16),
                       torch.zeros((pages, d)), torch.zeros((pages, d)),
                       torch.zeros((r, hkv, nb), dtype=torch.int32),
                       torch.full((r,), nb, dtype=torch.int32),
                       torch.full((r,), nb * b, dtype=torch.int64))
    q = torch.zeros((r, 4, d), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="ntokens"):
        paged.exact(q, kv, 2)

