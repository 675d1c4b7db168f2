"""The SG list ring protocol between GPU submitter waves and transfer waves,
checked on its state-machine model (tests/sg_ring_model.py; the kernels are
include/gfd/sg_device_primitives.h and include/gfd/sg_warp_spec.h).

- Every interleaving of a ring of 3 slots, 2 submitters and 2 transfer waves
  posting 7 lists (each slot reused twice) ends with every list landed
  exactly once, with lists dealt to submitters as the MoE kernel deals them
  and with list ids from a shared counter alike.
- The same search finds the deadlock when a transfer wave's claim store
  (sequence = 0) is not ordered before its release of `done`: the store lands
  after the slot's next list was committed and erases that commit.
- Random interleavings at the shape of the MoE session launch that once hung
  (1088 lists over the 512-slot ring, 64 submitters, 64 transfer waves),
  with actors of very different speeds, all end.
- The MoE kernel's current form when its lists fit the ring: list L placed
  at ring index L with no allocation or waits, and the transfer wave that
  lands the last list ending the launch (sg_stop_when_landed).  Every
  interleaving ends, also with the lander stop over a reused ring; without
  the submitter's own check of lists_done (all lists landed before stop_at
  was set) the search finds the launch that never ends."""
import pytest

from sg_ring_model import Model


@pytest.mark.parametrize("assign", ["mod", "shared"])
def test_no_interleaving_deadlocks_with_ordered_claim_stores(assign):
    states, problem = Model(3, 2, 2, 7, assign, "ordered").explore()
    assert problem is None, (problem[0], Model(3, 2, 2, 7, assign, "ordered").replay(problem[1])[1])
    assert states > 10_000


def test_unordered_claim_store_can_erase_the_next_commit():
    m = Model(3, 2, 2, 7, "mod", "reorderable")
    _, problem = m.explore()
    assert problem is not None and problem[0] == "deadlock"
    s, lines = m.replay(problem[1])
    # Stuck: some committed list was wiped before any wave saw it, and the
    # wave at list_known waits for it with nothing left to move.
    assert s.ld < m.total
    assert any(w[1] == s.lk for w in s.waves), "\n".join(lines)
    assert any(line.split()[0] == "wave" and "claim store" in line for line in lines)


@pytest.mark.parametrize("assign", ["mod", "shared"])
@pytest.mark.parametrize("seed", [1, 2, 3])
def test_full_size_launch_random_interleavings_end(assign, seed):
    steps, outcome = Model(512, 64, 64, 1088, assign, "ordered").simulate(seed)
    assert outcome == "ok", (assign, seed, steps)


@pytest.mark.parametrize("place,ring,total", [("fixed", 8, 7), ("alloc", 3, 7)])
def test_lander_stop_never_deadlocks(place, ring, total):
    m = Model(ring, 2, 2, total, "mod", "ordered", place=place, stop="lander")
    states, problem = m.explore()
    assert problem is None, (problem[0], m.replay(problem[1])[1])
    assert states > 1_000


def test_lander_stop_needs_the_submitters_own_check():
    m = Model(8, 2, 2, 3, "mod", "ordered", place="fixed", stop="lander_unchecked")
    _, problem = m.explore()
    assert problem is not None and problem[0] == "deadlock"
    s, lines = m.replay(problem[1])
    # Every list landed before stop_at was set, so no lander raised stop.
    assert s.ld == m.total and s.sa == m.total and not s.stop, "\n".join(lines)


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_moe_launch_with_fixed_places_random_interleavings_end(seed):
    steps, outcome = Model(512, 32, 32, 370, "mod", "ordered", place="fixed", stop="lander").simulate(seed)
    assert outcome == "ok", (seed, steps)
