"""bench.py's CPU baseline leg: every kind that cpu_baseline() can hand to the
subprocess parses and decodes on the host (no GPU), so the bench line's
cpu_baseline cannot silently come out null."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import bench  # noqa: E402


@pytest.fixture(scope="module")
def tiny_gguf(tmp_path_factory):
    from llama3pure_amd import synth
    g = synth.synthetic_model(dim=256, hidden=512, n_layers=2, n_heads=8, n_kv=2, vocab=512, ctx=128, seed=5)
    p = tmp_path_factory.mktemp("cpu_leg") / "tiny.gguf"
    p.write_bytes(bytes(g))
    return str(p)


def leg_kinds():
    """The kinds cpu_baseline() passes: the OpenMP line at the host's ISA
    level, the single-thread -O3 line, or the oracle when the reference
    was not built."""
    import oracle
    kinds = ["port"]
    if oracle.have_ref():
        kinds += ["o3", "omp_v4" if bench.host_has_avx512() else "omp"]
    return kinds


@pytest.mark.parametrize("kind", leg_kinds())
def test_cpu_leg_runs(tiny_gguf, kind):
    r = bench.run_cpu_leg(tiny_gguf, 0.05, kind, 2, 3)
    assert r is not None, f"cpu leg {kind} failed"
    assert r["tokens"] >= 1 and r["seconds"] > 0
    if kind.startswith("omp"):
        assert [g["shape"] for g in r["gemv"]] == [f"{n} {rows}x{cols}" for n, _, rows, cols in bench.GEMV_SHAPES]
