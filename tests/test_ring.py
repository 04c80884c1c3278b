"""The slice timer's ring on the CPU (bls_ring_*, beatlm_amd/csrc/ring.cpp):
the bookkeeping that decides which slot a frame's events use and when they
may be read, with no GPU in it. The cases follow the reference's own ring
tests (crates/beatlm/src/gpu/ring.rs:422-896) rule by rule: slots in order
with a cursor that waits on the oldest; a slot read only after its ticket came
back; a dropped ticket freeing its slot unread; invalidation; held slots and
verdicts; submission order. A dropped Rust `Ticket` or `Verdict` is
`drop_ticket` / `verdict(hold, False)` here."""

import threading

import pytest

from beatlm_amd import schedule as S
from beatlm_amd.schedule import (COLLECT_DROP, COLLECT_READ, COLLECT_WAIT, DONE_FAILED, DONE_OK, DONE_PENDING,
                                 PHASE_ENCODED, PHASE_FREE, PHASE_HELD, PHASE_INVALID, PHASE_RECORDING,
                                 PHASE_SUBMITTED, Ring)

READ = COLLECT_READ
WAIT = COLLECT_WAIT
DROP = COLLECT_DROP


def submit_one(ring):
    slot = ring.claim()
    return ring.submit(ring.encode(slot))


def hold_one(ring):
    slot = ring.claim()
    return ring.submit_held(ring.encode(slot))


def all_ok(_):
    return DONE_OK


def test_slots_are_handed_out_in_order_and_wrap():
    ring = Ring(3)
    for want in (0, 1, 2, 0):
        assert ring.claim() == want
        ring.release(want)


def test_a_busy_slot_is_refused_and_the_cursor_stays():
    ring = Ring(2)
    assert ring.claim() == 0
    assert ring.claim() == 1
    assert ring.claim() is None
    assert ring.claim() is None
    ring.release(0)
    assert ring.claim() == 0


def test_a_submitted_ticket_makes_its_slot_readable():
    ring = Ring(2)
    slot = ring.claim()
    assert ring.slots_in(PHASE_SUBMITTED) == []
    ticket = ring.encode(slot)
    assert ticket is not None and ticket & 0xFF == slot
    # Encoded, not handed back: in flight and unreadable.
    assert ring.phase(slot) == PHASE_ENCODED
    assert ring.in_flight() == 1
    assert ring.submit(ticket) == slot
    assert ring.slots_in(PHASE_SUBMITTED) == [slot]
    assert ring.in_flight() == 1
    ring.release(slot)
    assert ring.in_flight() == 0


def test_a_dropped_ticket_frees_its_slot_unread():
    ring = Ring(2)
    slot = ring.claim()
    S.drop_ticket(ring.encode(slot))
    assert ring.in_flight() == 0
    assert ring.slots_in(PHASE_SUBMITTED) == []
    assert ring.claim() == 1
    assert ring.reclaimed() == 1
    ring.release(1)
    assert ring.claim() == slot
    assert ring.slots_in(PHASE_SUBMITTED) == []


def test_a_ticket_from_an_earlier_lap_does_not_leak_into_the_next():
    ring = Ring(1)
    old = ring.encode(ring.claim())
    S.drop_ticket(old)
    ticket = ring.encode(ring.claim())
    assert ticket != old
    # The earlier lap's ticket reaches nothing: dropped again, or handed back.
    S.drop_ticket(old)
    assert ring.submit(old) is None
    assert ring.in_flight() == 1
    assert ring.submit(ticket) == 0
    assert ring.slots_in(PHASE_SUBMITTED) == [0]


def test_tickets_may_come_back_out_of_order():
    ring = Ring(3)
    first = ring.encode(ring.claim())
    second = ring.encode(ring.claim())
    third = ring.encode(ring.claim())
    assert ring.submit(third) == 2
    S.drop_ticket(first)
    assert ring.submit(second) == 1
    assert ring.slots_in(PHASE_SUBMITTED) == [1, 2]
    assert ring.in_flight() == 2
    # The dropped slot is free again and the cursor, back on it, takes it.
    assert ring.claim() == 0


def test_a_full_ring_refuses_until_a_ticket_is_dropped():
    ring = Ring(2)
    a = ring.encode(ring.claim())
    b = ring.encode(ring.claim())
    assert ring.claim() is None
    assert ring.in_flight() == 2
    # Dropping the one not at the cursor frees it, but the cursor waits on the oldest.
    S.drop_ticket(b)
    assert ring.in_flight() == 1
    assert ring.claim() is None
    S.drop_ticket(a)
    assert ring.claim() == 0
    assert ring.claim() == 1


def test_a_ticket_from_another_ring_is_refused_and_frees_its_own_slot():
    mine, theirs = Ring(2), Ring(2)
    held = mine.encode(mine.claim())
    foreign = theirs.encode(theirs.claim())
    assert mine.submit(foreign) is None
    assert mine.slots_in(PHASE_SUBMITTED) == []
    assert mine.in_flight() == 1
    assert theirs.slots_in(PHASE_SUBMITTED) == []
    assert theirs.in_flight() == 0
    # Spent: handed to its own ring afterwards it is refused there too.
    assert theirs.submit(foreign) is None
    assert mine.submit(held) == 0


def test_only_a_recording_slot_is_encoded():
    ring = Ring(2)
    assert ring.encode(0) is None
    slot = ring.claim()
    ticket = ring.encode(slot)
    assert ring.encode(slot) is None
    assert ring.submit(ticket) == slot
    assert ring.encode(slot) is None
    # A ticket comes back once.
    assert ring.submit(ticket) is None


def test_unknown_slots_are_ignored():
    ring = Ring(1)
    assert ring.encode(9) is None
    ring.release(9)
    assert ring.phase(9) is None
    assert ring.in_flight() == 0


def test_only_a_completed_submitted_slot_is_read():
    assert S.collect_action(PHASE_SUBMITTED, DONE_OK) == READ
    assert S.collect_action(PHASE_SUBMITTED, DONE_PENDING) == WAIT
    assert S.collect_action(PHASE_SUBMITTED, DONE_FAILED) == DROP
    assert S.collect_action(PHASE_INVALID, DONE_PENDING) == WAIT
    assert S.collect_action(PHASE_INVALID, DONE_OK) == DROP
    assert S.collect_action(PHASE_INVALID, DONE_FAILED) == DROP
    for phase in (PHASE_FREE, PHASE_RECORDING, PHASE_ENCODED, PHASE_HELD):
        for done in (DONE_PENDING, DONE_OK, DONE_FAILED):
            assert S.collect_action(phase, done) == WAIT, (phase, done)


def test_a_slot_invalidated_before_its_work_completes_waits_then_drops():
    ring = Ring(2)
    slot = submit_one(ring)
    assert ring.invalidate() == 1
    assert ring.phase(slot) == PHASE_INVALID
    # Still held: its events may yet be written.
    assert ring.in_flight() == 1
    assert ring.ready(lambda i: DONE_PENDING) == []
    assert ring.ready(all_ok) == [(slot, DROP)]
    ring.release(slot)
    assert ring.in_flight() == 0


def test_a_slot_invalidated_after_its_work_completed_is_still_dropped():
    ring = Ring(2)
    slot = submit_one(ring)
    assert ring.ready(all_ok) == [(slot, READ)]
    ring.invalidate()
    assert ring.ready(all_ok) == [(slot, DROP)]


def test_invalidation_spares_frames_not_yet_handed_back():
    ring = Ring(3)
    first = ring.encode(ring.claim())
    second = submit_one(ring)
    third = ring.claim()
    assert ring.invalidate() == 1
    assert ring.phase(second) == PHASE_INVALID
    assert ring.phase(third) == PHASE_RECORDING
    assert ring.submit(first) == 0
    assert ring.phase(0) == PHASE_SUBMITTED
    assert ring.submit(ring.encode(third)) == 2
    assert ring.slots_in(PHASE_SUBMITTED) == [0, 2]
    assert ring.slots_in(PHASE_INVALID) == [1]
    # Again: only what was submitted since moves.
    assert ring.invalidate() == 2
    assert ring.invalidate() == 0


def test_an_invalid_slot_holds_its_place_and_the_next_lap_is_readable():
    ring = Ring(2)
    a = submit_one(ring)
    b = submit_one(ring)
    ring.invalidate()
    assert ring.claim() is None
    ring.release(a)
    ring.release(b)
    again = submit_one(ring)
    assert again == a
    assert ring.phase(again) == PHASE_SUBMITTED
    assert ring.ready(all_ok) == [(again, READ)]
    assert submit_one(ring) == b
    assert ring.phase(b) == PHASE_SUBMITTED


def test_a_held_slot_waits_for_its_verdict_whatever_its_work_did():
    ring = Ring(2)
    slot, hold = hold_one(ring)
    assert ring.phase(slot) == PHASE_HELD
    assert ring.in_flight() == 1
    ring.settle()
    assert ring.phase(slot) == PHASE_HELD
    for done in (DONE_PENDING, DONE_OK, DONE_FAILED):
        assert ring.ready(lambda i, d=done: d) == []
    assert S.verdict(hold, True)
    # Nothing moves until the ring settles.
    assert ring.phase(slot) == PHASE_HELD
    ring.settle()
    assert ring.phase(slot) == PHASE_SUBMITTED
    assert ring.ready(all_ok) == [(slot, READ)]


def test_a_rejected_or_unanswered_verdict_invalidates_only_its_own_slot():
    ring = Ring(3)
    rejected, r_hold = hold_one(ring)
    dropped, d_hold = hold_one(ring)
    accepted, a_hold = hold_one(ring)
    assert S.verdict(r_hold, False)
    assert S.verdict(d_hold, False)  # the C form of dropping a Verdict unsettled
    assert S.verdict(a_hold, True)
    ring.settle()
    assert ring.phase(rejected) == PHASE_INVALID
    assert ring.phase(dropped) == PHASE_INVALID
    assert ring.phase(accepted) == PHASE_SUBMITTED
    assert ring.ready(all_ok) == [(rejected, DROP), (dropped, DROP), (accepted, READ)]
    # A second verdict on a settled hold reaches nothing.
    assert not S.verdict(a_hold, False)


def test_a_later_frame_waits_while_an_earlier_one_is_held():
    ring = Ring(3)
    earlier, hold = hold_one(ring)
    later, later_hold = hold_one(ring)
    S.verdict(later_hold, True)
    ring.settle()
    assert ring.phase(later) == PHASE_SUBMITTED
    assert ring.ready(all_ok) == []
    ring.settle()
    assert ring.ready(all_ok) == []
    S.verdict(hold, True)
    ring.settle()
    assert ring.ready(all_ok) == [(earlier, READ), (later, READ)]


def test_a_later_frame_waits_while_an_earlier_one_is_running():
    ring = Ring(3)
    earlier = submit_one(ring)
    later = submit_one(ring)

    def pending(p):
        return lambda i: DONE_PENDING if i == p else DONE_OK

    assert ring.ready(pending(earlier)) == []
    assert ring.ready(pending(later)) == [(earlier, READ)]
    assert ring.ready(all_ok) == [(earlier, READ), (later, READ)]


def test_a_rejected_earlier_frame_holds_back_nothing():
    ring = Ring(3)
    earlier, hold = hold_one(ring)
    later, later_hold = hold_one(ring)
    S.verdict(later_hold, True)
    S.verdict(hold, False)
    ring.settle()
    assert ring.ready(all_ok) == [(earlier, DROP), (later, READ)]
    # Not even while its events are pending: it will never be read.
    assert ring.ready(lambda i: DONE_PENDING if i == earlier else DONE_OK) == [(later, READ)]
    ring.release(earlier)
    assert ring.ready(all_ok) == [(later, READ)]


def test_a_failed_earlier_frame_holds_back_nothing():
    ring = Ring(3)
    earlier = submit_one(ring)
    later = submit_one(ring)
    assert ring.ready(lambda i: DONE_FAILED if i == earlier else DONE_OK) == [(earlier, DROP), (later, READ)]


def test_a_frame_held_later_holds_back_only_what_follows_it():
    ring = Ring(3)
    earlier = submit_one(ring)
    held, _hold = hold_one(ring)
    later = submit_one(ring)
    assert held == 1
    assert ring.ready(all_ok) == [(earlier, READ)]
    assert ring.phase(later) == PHASE_SUBMITTED


def test_unheld_frames_are_ready_in_submission_order_as_they_complete():
    ring = Ring(3)
    a = ring.encode(ring.claim())
    b = ring.encode(ring.claim())
    c = ring.encode(ring.claim())
    c = ring.submit(c)
    a = ring.submit(a)
    b = ring.submit(b)
    assert ring.ready(lambda i: DONE_PENDING) == []
    assert ring.ready(all_ok) == [(c, READ), (a, READ), (b, READ)]

    def upto(slot):
        return lambda i: DONE_OK if i in (slot, c) else DONE_PENDING

    assert ring.ready(upto(c)) == [(c, READ)]
    ring.release(c)
    assert ring.ready(upto(a)) == [(a, READ)]
    ring.release(a)
    assert ring.ready(all_ok) == [(b, READ)]


def test_a_held_slot_keeps_the_cursor_as_a_submitted_one_does():
    ring = Ring(2)
    first, hold = hold_one(ring)
    submit_one(ring)
    assert ring.claim() is None
    S.verdict(hold, True)
    ring.settle()
    ring.release(first)
    assert ring.claim() == first


def test_invalidation_takes_held_slots_and_a_late_verdict_reaches_nothing():
    ring = Ring(1)
    slot, late = hold_one(ring)
    assert ring.invalidate() == 1
    assert ring.phase(slot) == PHASE_INVALID
    ring.release(slot)
    again, hold = hold_one(ring)
    assert again == slot
    assert not S.verdict(late, True)
    ring.settle()
    assert ring.phase(again) == PHASE_HELD
    assert S.verdict(hold, False)
    ring.settle()
    assert ring.phase(again) == PHASE_INVALID


def test_a_held_ticket_from_another_ring_is_refused():
    mine, theirs = Ring(1), Ring(1)
    foreign = theirs.encode(theirs.claim())
    assert mine.submit_held(foreign) is None
    assert mine.slots_in(PHASE_HELD) == []
    assert theirs.in_flight() == 0


def test_a_zero_depth_ring_still_has_one_slot():
    ring = Ring(0)
    assert ring.depth() == 1
    assert ring.claim() == 0
    assert ring.claim() is None


# ---- beyond the reference's cases: what the C form adds ----


def test_a_ring_deeper_than_the_maximum_is_refused():
    with pytest.raises(S.ScheduleError):
        Ring(S.RING_MAX_DEPTH + 1)
    assert Ring(S.RING_MAX_DEPTH).depth() == S.RING_MAX_DEPTH


def test_tickets_and_verdicts_of_a_freed_ring_reach_nothing():
    ring = Ring(2)
    ticket = ring.encode(ring.claim())
    _, hold = hold_one(ring)
    ring.close()
    S.drop_ticket(ticket)
    assert not S.verdict(hold, True)
    other = Ring(2)
    assert other.submit(ticket) is None
    assert other.in_flight() == 0


def test_tickets_may_be_dropped_and_verdicts_given_from_other_threads():
    ring = Ring(4)
    tickets = [ring.encode(ring.claim()) for _ in range(2)]
    holds = [hold_one(ring) for _ in range(2)]
    results = []
    threads = [threading.Thread(target=S.drop_ticket, args=(t,)) for t in tickets]
    threads += [threading.Thread(target=lambda h=h: results.append(S.verdict(h, True))) for _, h in holds]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert results == [True, True]
    assert ring.in_flight() == 2
    ring.settle()
    assert ring.ready(all_ok) == [(holds[0][0], READ), (holds[1][0], READ)]
    assert ring.claim() == 0  # the cursor wrapped back to a dropped slot
    assert ring.reclaimed() == 2


def test_a_frame_loop_over_many_laps_reads_every_frame_once_in_order():
    """Frames 0..299 through a ring of 3 the way the timer drives it: claim,
    encode, hand back (every 7th dropped, every 5th held and judged two frames
    later, every 11th invalidated after submission), collect what is ready,
    with most frames' work done a frame later and every 4th frame's four
    frames later (so some frames find their slot busy). No frame is read
    twice, out of submission order, after its ticket was dropped or after its
    verdict rejected it."""
    ring = Ring(3)
    frame_of = {}
    read, dropped, skipped = [], [], 0
    pending_verdicts = []  # (due frame, hold, accept)
    running = {}  # slot -> the frame at whose start its work has completed
    for f in range(300):
        for due, hold, accept in [p for p in pending_verdicts if p[0] == f]:
            S.verdict(hold, accept)
            pending_verdicts.remove((due, hold, accept))
        ring.settle()
        for slot, act in ring.ready(lambda i: DONE_PENDING if running.get(i, 0) > f else DONE_OK):
            (read if act == READ else dropped).append(frame_of[slot])
            ring.release(slot)
        slot = ring.claim()
        if slot is None:
            skipped += 1
            continue
        frame_of[slot] = f
        ticket = ring.encode(slot)
        if f % 7 == 3:
            S.drop_ticket(ticket)
            continue
        if f % 5 == 1:
            s, hold = ring.submit_held(ticket)
            pending_verdicts.append((f + 2, hold, f % 10 != 1))
        else:
            ring.submit(ticket)
        running[slot] = f + (4 if f % 4 == 0 else 1)
        if f % 11 == 6:
            ring.invalidate()
    assert read == sorted(read) and len(set(read)) == len(read)
    for f in read:
        assert f % 7 != 3, f"frame {f} was dropped and still read"
        assert f % 10 != 1, f"frame {f} was rejected and still read"
    assert not set(read) & set(dropped)
    assert len(read) > 100 and skipped > 0
