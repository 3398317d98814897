"""The conv-fused decode's last-arriver ticket (gdn_decode.hip, count_in): each workgroup of
a k-head group of `group` workgroups counts itself in with a wrapping increment (the
hardware's atomic inc: the ticket becomes 0 when it held group - 1, else its value + 1,
returning the previous value); the one that receives group - 1 writes the shared q/k conv
state.  Emulated here with random arrival orders: exactly the last arriver writes, tickets
return to zero after every launch, and a batch that repeats a conv slot or two interleaved
launches on the same slots (both outside the op's contract) leave the tickets at zero for
the next launch.  The previous protocol (writer on an exact match, then a store of 0) is
shown to strand a count after a repeated slot (the reason for the change)."""

from __future__ import annotations

import random


def wrapping_increment(tickets, key, group):
    old = tickets.get(key, 0)
    tickets[key] = 0 if old >= group - 1 else old + 1
    return old


def run_launch(tickets, arrivals, group, protocol="wrapping"):
    """arrivals: the (key, workgroup) sequence of one launch's count-ins.  Returns the
    workgroups that write (by the protocol's rule) in arrival order."""
    writers = []
    for key, workgroup in arrivals:
        if protocol == "wrapping":
            old = wrapping_increment(tickets, key, group)
            if old == group - 1:
                writers.append((key, workgroup))
        else:  # exact match on group - 1, then a store of 0 by the writer (at its end)
            old = tickets.get(key, 0)
            tickets[key] = old + 1
            if old == group - 1:
                writers.append((key, workgroup))
                tickets[key] = 0
    return writers


def test_last_arriver_writes_and_tickets_return_to_zero():
    rng = random.Random(0)
    for group in (2, 3, 4, 6):
        tickets = {}
        for launch in range(50):
            keys = rng.sample(range(40), 8)  # distinct conv slots (x k-heads)
            arrivals = [(k, w) for k in keys for w in range(group)]
            rng.shuffle(arrivals)
            writers = run_launch(tickets, arrivals, group)
            assert sorted(k for k, _ in writers) == sorted(keys)
            for key, workgroup in writers:  # the writer is the key's last arrival
                last = [w for k, w in arrivals if k == key][-1]
                assert workgroup == last
            assert all(v == 0 for v in tickets.values())


def test_repeated_slot_or_interleaved_launches_leave_tickets_at_zero():
    rng = random.Random(1)
    for group in (2, 3):
        tickets = {}
        # a batch repeating slot 5 (two requests on one conv slot)
        arrivals = [(5, w) for w in range(2 * group)] + [(k, w) for k in (1, 2) for w in range(group)]
        rng.shuffle(arrivals)
        run_launch(tickets, arrivals, group)
        assert all(v == 0 for v in tickets.values())
        # two launches on the same slots, interleaved (e.g. two streams)
        a = [(k, ("a", w)) for k in (3, 4) for w in range(group)]
        b = [(k, ("b", w)) for k in (3, 4) for w in range(group)]
        merged = a + b
        rng.shuffle(merged)
        run_launch(tickets, merged, group)
        assert all(v == 0 for v in tickets.values())
        # a clean launch afterwards: exactly the last arriver of each key writes
        arrivals = [(k, w) for k in (3, 4, 5) for w in range(group)]
        rng.shuffle(arrivals)
        writers = run_launch(tickets, arrivals, group)
        for key, workgroup in writers:
            assert workgroup == [w for k, w in arrivals if k == key][-1]
        assert len(writers) == 3


def test_previous_protocol_strands_a_count_after_a_repeated_slot():
    tickets = {}
    group = 2
    arrivals = [(5, 0), (5, 1), (5, 2), (5, 3)]  # two requests on slot 5, in order
    # exact match + store 0: 0, 1 (writes, stores 0), 0, 1 (writes, stores 0) -> fine in order,
    # but with the second request's first arrival between the writer's count-in and its
    # store (the store comes at the writer's end), the count is stranded:
    tickets = {5: 0}
    old0 = tickets[5]; tickets[5] += 1            # request A, wg 0 -> 0
    old1 = tickets[5]; tickets[5] += 1            # request A, wg 1 -> 1: writer
    old2 = tickets[5]; tickets[5] += 1            # request B, wg 0 -> 2 (before A's store)
    tickets[5] = 0                                # A's writer stores 0 at its end
    old3 = tickets[5]; tickets[5] += 1            # request B, wg 1 -> 0: nobody else writes
    assert (old0, old1, old2, old3) == (0, 1, 2, 0)
    assert tickets[5] == 1                        # stranded: the next launch's first arriver
    writers = run_launch(tickets, [(5, 0), (5, 1)], group, protocol="exact")
    assert writers == [(5, 0)]                    # writes before the other has read
    del arrivals
