"""bench.py's per-call traffic and VALU figures must be the ones the committed rocprof summaries state.

The counters cannot be read from inside the bench process, so ``bench.MEASURED_TRAFFIC`` and
``bench.MEASURED_VALU`` are tables; this test keeps them tied to ``profiles/``: every figure
appears in its source summary, and for summaries whose table has a ``call`` column the figure is
the sum of that call's rows (dispatch rows marked ``x 2 per call`` count twice).
"""

import re
from pathlib import Path

import pytest

import bench

ROOT = Path(__file__).resolve().parents[1]


def _num(s: str) -> float:
    return float(s.replace(",", ""))


def _call_rows(text: str):
    """(kernel, call, per-call multiplicity, numeric columns) of a summary table with a call column."""
    rows = []
    header = None
    for line in text.splitlines():
        if not line.startswith("|"):
            continue
        cells = [c.strip() for c in line.strip("|").split("|")]
        if header is None:
            header = cells
            continue
        if set(line) <= set("|-"):
            continue
        if "call" not in header:
            return []
        rec = dict(zip(header, cells))
        mult = 2 if "x 2 per call" in rec["kernel"] else 1
        rows.append((rec["kernel"], rec["call"], mult, rec))
    return rows


def _mentions(text: str, value: float, decimals: int) -> bool:
    plain = f"{value:.{decimals}f}"
    grouped = f"{value:,.{decimals}f}"
    return plain in text or grouped in text


@pytest.mark.parametrize("key", list(bench.MEASURED_TRAFFIC))
def test_traffic_table_matches_profiles(key):
    for phase, (nbytes, source) in bench.MEASURED_TRAFFIC[key].items():
        text = (ROOT / source).read_text()
        mb = nbytes / 1e6
        assert _mentions(text, mb, 1), f"{key} {phase}: {mb:.1f} MB not stated in {source}"
        rows = _call_rows(text)
        if rows:
            total = sum(
                mult * (_num(r["read MB (scaled)"]) + _num(r["written MB (scaled)"]))
                for _, call, mult, r in rows
                if call == phase
            )
            assert abs(total - mb) < 0.2, f"{key} {phase}: rows of {source} sum to {total:.1f} MB, table says {mb:.1f}"


@pytest.mark.parametrize("key", list(bench.MEASURED_VALU))
def test_valu_table_matches_profiles(key):
    for phase, (quads, source) in bench.MEASURED_VALU[key].items():
        text = (ROOT / source).read_text()
        assert _mentions(text, quads, 0), f"{key} {phase}: {quads} not stated in {source}"
        rows = _call_rows(text)
        if rows:
            col = next(c for c in rows[0][3] if c.startswith("SQ_ACTIVE_INST_VALU"))
            total = sum(mult * _num(r[col]) for _, call, mult, r in rows if call == phase)
            assert total == quads, f"{key} {phase}: rows of {source} sum to {total}, table says {quads}"


def test_profiles_name_their_command():
    """Every summary the tables cite gives the rocprofv3 command that produced it."""
    sources = {src for tbl in (bench.MEASURED_TRAFFIC, bench.MEASURED_VALU) for v in tbl.values() for _, src in v.values()}
    for source in sources:
        text = (ROOT / source).read_text()
        assert re.search(r"rocprofv3 .*-- python3 bench\.py", text), source
