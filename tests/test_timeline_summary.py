"""CPU test of the timeline tool's summary (ffa_mi355x.timeline.summarize) on synthetic stamps."""
import numpy as np

from ffa_mi355x import timeline as TL


def _stamps(nwg=8, seed=0):
    """4 waves per workgroup; stamps in 100 MHz ticks, increasing along the path; waves 0 of odd
    workgroups refine one chunk each (word 13), the workgroup's kept chunks in word 14."""
    rng = np.random.default_rng(seed)
    st = np.zeros((nwg * 4, 16), dtype=np.int64)
    base = 1_000_000
    for w in range(nwg * 4):
        t = base + np.cumsum(rng.integers(5, 50, size=13))
        st[w, :13] = t
        wg = w // 4
        if wg % 2 == 1 and w % 4 == 0:
            st[w, 13] = 1
        st[w, 14] = 1 if wg % 2 == 1 else 0
        st[w, 15] = ((wg % 8) << 32) | ((wg % 4) << 8)  # XCC_ID << 32 | HW_ID (CU id bits 8-11)
    return st


def test_summarize_prints_every_point_and_the_workgroup_tables(capsys):
    st = _stamps()
    TL.summarize(st, TL.POINTS["config2"], per_wg=True, exact_points=TL.EXACT_POINTS["config2"])
    out = capsys.readouterr().out
    for name in TL.POINTS["config2"]:
        assert name in out
    assert "workgroups with 0 kept chunks" in out and "workgroups with 1 kept chunks" in out
    assert "per XCD" in out
    # medians are non-negative microseconds from the first wave's start
    first = out.splitlines()[1].split()
    assert float(first[-3]) >= 0.0


def test_summarize_skips_points_a_layout_does_not_stamp(capsys):
    st = _stamps()
    st[:, 1] = 0  # the contiguous q2 layout records no page-id point
    TL.summarize(st, TL.POINTS["config2ref"], per_wg=True, exact_points=TL.EXACT_POINTS["config2ref"])
    out = capsys.readouterr().out
    assert "operands built" in out
    table = out.split("waves with")[0].splitlines()[1:]
    assert len(table) == len([n for n in TL.POINTS["config2ref"] if n != "-"])
    for line in table:  # a zero stamp would print as a large negative time
        assert all(float(x) >= 0.0 for x in line.split()[-3:]), line
