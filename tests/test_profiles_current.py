"""The committed rocprofv3 summaries under ``profiles/`` were taken on the
kernel sources in the tree, and name the kernels ``bench.py`` reads.

``bench.py`` takes ``roofline.traffic`` from the PMC table and refuses a
table whose recorded source hash differs from the sources' own; these checks
make the same comparison on the CPU, so a kernel edit that was not
re-profiled fails here rather than surfacing as a null ``traffic`` field.
"""
import importlib.util
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def _bench():
    spec = importlib.util.spec_from_file_location("pkda_bench_module", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_every_profile_records_the_current_source_hash():
    bench = _bench()
    current = bench.kernel_source_hash()
    found = 0
    for md in sorted((ROOT / "profiles").glob("*.md")):
        m = re.search(r"^source hash: `([0-9a-f]+)`", md.read_text(), re.M)
        if m:
            found += 1
            assert m.group(1) == current, f"{md.name} was profiled on sources {m.group(1)}, the tree is {current}"
    assert found >= 1


def test_bench_kernels_have_traffic_rows():
    bench = _bench()
    names = set(bench.STAGE_KERNEL.values()) | set(bench.PRODUCTION_STAGE_KERNEL.values())
    for name in sorted(names):
        t = bench.profiled_traffic(name)
        assert t is not None, f"no PMC traffic row for {name}"
        assert not t.get("stale"), t
        assert t["read_MiB"] > 0 and t["bytes"] > 0
