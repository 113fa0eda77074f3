"""The macro-tile kernel's scale ring, on a model of its schedule (CPU only).

gemm_tile keeps the e8m0 scale rows of k-groups (4 slabs each) in an LDS ring of R slots. During
slab kt, after its barrier, a wave refills the stage of slab kt-1 with slab kt + NS - 1 (kt + NS on
the deep-tile path, WM >= 3) and, when that slab starts a k-group, the fill also carries the rows of
the k-group after it into slot (group % R). Such a fill may land at any moment until the wait before
the first slab that reads it. Slab j reads its group's slot after barrier j (the deep-tile path
reads a group's rows once, at slab 4g - 1, after that slab's barrier), and those reads complete
before barrier j + 1. The kernel sizes R with ring_slots(NS) so that NS < 4 R - 6, checked at
compile time (csrc/w4a8_gemm_tile.hip); this test checks that condition against the schedule:
no fill may land on a slot that a slab of another k-group reads."""
import pytest


def conflicts(ns: int, r: int, deep: bool, kt4: int = 64) -> int:
    reads = {}                                     # phase -> {(slot, group)}; phase 2j+1 = after barrier j
    fills = []                                     # (issue phase, last landing phase, slot, group)
    for kt in range(kt4):
        if deep:
            if kt % 4 == 3:
                g = (kt + 1) // 4
                reads.setdefault(2 * kt + 1, set()).add((g % r, g))
            s = kt + ns
            if s % 4 == 0:
                gp = s // 4 + 1
                fills.append((2 * kt + 1, 2 * (4 * gp - 1) + 1, gp % r, gp))
        else:
            g = kt // 4
            reads.setdefault(2 * kt + 1, set()).add((g % r, g))
            s = kt + ns - 1
            if s % 4 == 0:
                gp = s // 4 + 1
                fills.append((2 * kt + 1, 2 * (4 * gp) + 1, gp % r, gp))
    bad = 0
    for issue, land_by, slot, gp in fills:
        for ph in range(issue, land_by + 1):
            bad += sum(1 for sl, g in reads.get(ph, ()) if sl == slot and g != gp)
    return bad


@pytest.mark.parametrize("ns", range(2, 17))
def test_condition_is_exactly_what_the_schedule_needs(ns):
    smallest = next(r for r in range(2, 12) if conflicts(ns, r, deep=False) == 0)
    assert all(conflicts(ns, r, deep=False) == 0 for r in range(smallest, smallest + 3))
    # NS < 4 R - 6 picks the same smallest ring (at least 3 slots) for the head-barrier path
    assert max(3, smallest) == next(r for r in range(3, 12) if ns < 4 * r - 6)
    # the deep-tile path (scales read once per group) needs no more
    assert conflicts(ns, max(3, smallest), deep=True) == 0


def test_three_slots_stop_at_five_stages():
    assert conflicts(5, 3, deep=False) == 0
    assert conflicts(6, 3, deep=False) > 0
    assert conflicts(8, 3, deep=False) > 0         # the depth the decode band plans
