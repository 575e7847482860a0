"""Model check (CPU) of the split combine's arrival word, the protocol of
`slice_arrive` in include/sde/attention_device.hpp, over every interleaving
of small cases.

The word (zero at rest): bits 0-7 count the partitions' arrivals, bits 8-15
the waiting workgroups' final operations, bits 16-23 their give-up bits.
Workgroups arrive in any order; the one that arrives s places before the
last (1 <= s < n_slices) waits and then either sees every arrival in (its
final operation adds 1 << 8) or gives up at any moment after its own
arrival (it adds 1 << 8 plus its give-up bit).  Checked for every arrival
order and every placement of the final operations: each slice is combined
exactly once (the last arrival takes slice 0 and the slices its arrival
saw given up; a waiter takes its own slice unless it gave up before the
last arrival), the word is back at zero at the end, and no operation
touches it after its reset.  The GPU test
test_gpu_attention.py::test_split_combine_slices_and_their_fallback runs
the device code with waits that give up at once.
"""
import itertools

import pytest


def run(n_parts, n_slices, order, finals, planted=False):
    """order: arrival order; finals: workgroup -> (kind, time), kind 'pass'
    (saw every arrival) or 'give' (gave up); arrivals happen at times 0..n-1.
    Returns the combined slices, the final word and whether an operation
    followed the reset, or None for an impossible interleaving.  planted:
    the unsplit combine's rule (the last arrival clears the word at once),
    a mistake the checks must catch."""
    want = n_parts
    last_op = want | ((n_slices - 1) << 8)
    W = 0
    done = []
    reset = False
    after_reset = False
    rank = {wg: n_parts - 1 - i for i, wg in enumerate(order)}
    events = [(i, 0, "arrive", wg) for i, wg in enumerate(order)]
    events += [(t, 1, kind, wg) for wg, (kind, t) in finals.items()]
    arrived = 0
    for _, _, kind, wg in sorted(events):
        after_reset |= reset
        if kind == "arrive":
            prev = W
            W += 1
            arrived += 1
            assert (prev & 0xFF) < want
            if n_parts - 1 - (prev & 0xFF) == 0:  # the last arrival
                if (W & 0xFFFF) == last_op or planted:
                    W, reset = 0, True
                done.append(0)
                done += [s for s in range(1, 8) if (prev >> (16 + s)) & 1]
        else:
            if kind == "pass" and (arrived < n_parts or (planted and reset and W == 0)):
                return None  # (a waiter cannot see every arrival in a cleared word)
            r = rank[wg]
            add = (1 << 8) | (0 if kind == "pass" else 1 << (16 + r))
            old = W
            W += add
            if (W & 0xFFFF) == last_op:
                W, reset = 0, True
            if kind == "pass" or (old & 0xFF) >= want:
                done.append(r)
    return sorted(done), W, after_reset


@pytest.mark.parametrize("n_parts", [2, 3, 4, 5])
def test_every_interleaving_combines_each_slice_once_and_resets(n_parts):
    checked = 0
    for n_slices in range(2, min(n_parts, 4) + 1):
        for order in itertools.permutations(range(n_parts)):
            at = {wg: i for i, wg in enumerate(order)}
            waiters = [wg for i, wg in enumerate(order) if 1 <= n_parts - 1 - i < n_slices]
            options = []
            for wg in waiters:
                opts = [("give", t + 0.5) for t in range(at[wg], n_parts - 1)]
                opts += [(k, n_parts - 1 + d) for k in ("pass", "give") for d in (0.25, 0.75)]
                options.append(opts)
            for combo in itertools.product(*options):
                r = run(n_parts, n_slices, list(order), dict(zip(waiters, combo)))
                if r is None:
                    continue
                done, word, after_reset = r
                assert done == list(range(n_slices)), (order, combo)
                assert word == 0 and not after_reset, (order, combo)
                checked += 1
    assert checked > 0


@pytest.mark.parametrize("n_parts", [8, 9, 16, 64])
def test_sampled_interleavings_up_to_eight_slices(n_parts):
    """16-row groups combine in up to eight 2-row slices (the give-up bits
    track ranks 1-7): seeded random arrival orders and final operations."""
    import random
    rng = random.Random(n_parts)
    checked = 0
    for n_slices in range(5, min(n_parts, 8) + 1):
        for _ in range(400):
            order = list(range(n_parts))
            rng.shuffle(order)
            at = {wg: i for i, wg in enumerate(order)}
            finals = {}
            for i, wg in enumerate(order):
                if 1 <= n_parts - 1 - i < n_slices:
                    opts = [("give", t + 0.5) for t in range(at[wg], n_parts - 1)]
                    opts += [(k, n_parts - 1 + d) for k in ("pass", "give") for d in (0.25, 0.75)]
                    finals[wg] = rng.choice(opts)
            r = run(n_parts, n_slices, order, finals)
            if r is None:
                continue
            done, word, after_reset = r
            assert done == list(range(n_slices)), (order, finals)
            assert word == 0 and not after_reset, (order, finals)
            checked += 1
    assert checked > 100


def test_a_wrong_reset_rule_is_caught():
    """The checks have teeth: with the last arrival clearing the word at
    once, a waiter polling for every arrival can only give up, and its
    final operation lands on a cleared word."""
    caught = 0
    order = [0, 1, 2]  # workgroup 1 arrives second: it waits for slice 1
    for kind, t in [("give", 2.25), ("give", 2.75)]:  # after the last arrival
        done, word, after_reset = run(3, 2, order, {1: (kind, t)}, planted=True)
        caught += done != [0, 1] or word != 0 or after_reset
        assert run(3, 2, order, {1: (kind, t)}) == ([0, 1], 0, False)
    assert caught == 2
