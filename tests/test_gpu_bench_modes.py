"""bench.py's table modes run end to end on small shapes: `--row-scaling` times every kernel it
names at every row count and reports what the dweight reduction adds.  Only the table's shape is
checked (timings are the bench's business, not a pass/fail criterion)."""

import re

import pytest

pytestmark = pytest.mark.gpu


def test_row_scaling_table_small():
    import bench

    rows = (1024, 2048)
    table = bench.row_scaling(d=4096, rows_list=rows, rounds=1)
    lines = table.splitlines()
    kernels = ("forward", "2R2W probe", "backward", "backward, no dweight", "2R1W probe",
               "2R1W best shape")
    for name in kernels:
        row = [ln for ln in lines if ln.startswith(f"| {name} |")]
        assert len(row) == 1, name
        vals = [float(v) for v in re.findall(r"\d+\.\d+", row[0])]
        assert len(vals) == len(rows) and all(v > 0 for v in vals), row[0]
    cost = [ln for ln in lines if re.match(r"\| (1024|2048) \|", ln)]
    assert len(cost) == len(rows)
    for ln in cost:
        float(ln.split("|")[2])  # a number, whatever its value
