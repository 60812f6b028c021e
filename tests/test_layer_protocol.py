"""The fused decode layer's hand-over protocol (k_layer_decode), modelled on
the CPU: leader election per XCD, the leader's wait for every gate/up flag,
the followers' wait for their XCD's flag line, and the lockstep counters
across consecutive launches.

The model follows the kernel's steps one to one (layer_kernels.h):
  gate/up workgroup g: runs, then sync[g] = target;
  down workgroup j on XCD x: ticket = exchange(tickets[x], target); stages
    its weights; if ticket != target it leads: waits until every gate/up
    flag == target, then stores target in line[x]; otherwise it waits until
    line[x] == target.
Workgroups are dispatched in id order into a bounded number of slots
(co-residency is not assumed) and advanced in a seeded random interleaving.
Every placement the dispatcher could produce is driven through it: all down
workgroups on one XCD, XCDs left empty, round-robin, random.  A run that
stops advancing is a hang.  The planted fault, the rule the kernel used to
follow (down workgroups 0-7 lead), must hang on some of these placements, so
the model can tell the two rules apart."""
from __future__ import annotations

import random

import pytest

XCDS = 8


def run_launches(placements, n_g, slots, seed, rule="ticket", launches=3):
    """Drive `launches` consecutive launches; placements[l][j] is down
    workgroup j's XCD in launch l.  Returns the number of launches that
    completed (a launch that stops advancing ends the run)."""
    rnd = random.Random(seed)
    tickets = [0] * XCDS
    lines = [0] * XCDS
    flags = [0] * n_g
    for launch in range(launches):
        target = launch + 1
        place = placements[launch % len(placements)]
        n_d = len(place)
        pending = list(range(n_g + n_d))         # dispatch order: gate/up ids first
        running = {}
        done = 0
        stalled = 0
        while done < n_g + n_d:
            while pending and len(running) < slots:   # the dispatcher fills free slots in id order
                b = pending.pop(0)
                running[b] = {"step": 0}
            b = rnd.choice(sorted(running))
            st = running[b]
            progressed = False
            if b < n_g:                                    # gate/up: two steps of work, then its flag
                st["step"] += 1
                progressed = True
                if st["step"] == 2:
                    flags[b] = target
                    del running[b]
                    done += 1
            else:
                j = b - n_g
                x = place[j]
                if st["step"] == 0:                        # arrival: the ticket
                    if rule == "ticket":
                        old, tickets[x] = tickets[x], target
                        st["leader"] = old != target
                    else:                                  # the fault: workgroups 0-7 lead
                        st["leader"] = j < XCDS or n_d <= XCDS
                    st["step"] = 1
                    progressed = True
                elif st["step"] == 1:                      # staging
                    st["step"] = 2
                    progressed = True
                elif st["leader"]:
                    if all(f == target for f in flags):
                        lines[x] = target
                        del running[b]
                        done += 1
                        progressed = True
                elif lines[x] == target:
                    del running[b]
                    done += 1
                    progressed = True
            stalled = 0 if progressed else stalled + 1
            if stalled > 200 * (len(running) + 1):
                return launch                              # nothing can advance: a hang
    return launches


def placements_for(n_d, rnd):
    yield [0] * n_d                                        # every down workgroup on one XCD
    yield [j % 8 for j in range(n_d)]                      # one per XCD in turn
    yield [j % 3 for j in range(n_d)]                      # five XCDs without any
    yield [7 - (j % 2) for j in range(n_d)]
    yield [1 + (j >= 8) * (j % 7) for j in range(n_d)]     # workgroups 0-7 on XCD 1 only
    for _ in range(6):
        yield [rnd.randrange(XCDS) for _ in range(n_d)]


@pytest.mark.parametrize("n_g,n_d", [(60, 23), (120, 16), (8, 5), (30, 64)])
@pytest.mark.parametrize("slots", [1, 4, 32, 10_000])
def test_every_placement_completes_with_one_leader_per_xcd(n_g, n_d, slots):
    rnd = random.Random(n_g * 1000 + n_d + slots)
    for place in placements_for(n_d, rnd):
        for seed in range(3):
            assert run_launches([place], n_g, slots, seed) == 3, (place, slots, seed)


def test_consecutive_launches_with_different_placements_and_grids():
    rnd = random.Random(5)
    for rep in range(20):
        n_d = rnd.choice([5, 16, 23])
        places = [[rnd.randrange(XCDS) for _ in range(n_d)] for _ in range(4)]
        assert run_launches(places, 40, rnd.choice([2, 16, 1000]), rep, launches=8) == 8


def test_election_gives_exactly_one_leader_per_occupied_xcd():
    rnd = random.Random(11)
    for rep in range(200):
        n_d = rnd.randrange(1, 40)
        place = [rnd.randrange(XCDS) for _ in range(n_d)]
        tickets = [rnd.randrange(5)] * XCDS                 # the previous launch's number
        target = 5 + rep
        order = list(range(n_d))
        rnd.shuffle(order)
        leaders = {}
        for j in order:
            old, tickets[place[j]] = tickets[place[j]], target
            if old != target:
                leaders.setdefault(place[j], []).append(j)
        assert sorted(leaders) == sorted(set(place))
        assert all(len(v) == 1 for v in leaders.values())


def test_the_fixed_leader_rule_hangs_where_a_placement_leaves_an_xcd_without_one():
    """The planted fault: leaders fixed as down workgroups 0-7.  With all of
    them on one XCD, the other XCDs' followers never see their flag line."""
    n_d = 23
    assert run_launches([[1 + (j >= 8) * (j % 7) for j in range(n_d)]], 60, 10_000, 0, rule="fixed") == 0
    assert run_launches([[j % 8 for j in range(n_d)]], 60, 10_000, 0, rule="fixed") == 3
