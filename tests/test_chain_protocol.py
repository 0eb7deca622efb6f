"""CPU model of the chain hand-off protocol of the chained solves (lucid_fwd.hip
lucid_precond_fwd_kernel, lucid_bwd.hip lucid_precond_bwd_col_kernel, path_fwd.hip /
path_bwd.hip chains; waits in mfma.h wait_counter_gt).

Model: workgroup ids are dispatched in increasing order onto a limited number of resident
slots; workgroup id owns chain block i = id // BH of head bh = id % BH.  Block i first reads
every earlier block j < i (it may read block j only once the head's counter exceeds j: the
producer writes block j, then publishes), then writes its own block and publishes
counter = i + 1.  Waits poll the counter; a bounded wait gives up after `limit` polls, sets
the error flag and carries on.  Interleavings are drawn at random.
"""
import random

import pytest


def simulate(n_blocks, BH, slots, seed, limit=None, broken=None, max_steps=200_000):
    """Run the protocol; returns (finished, read_before_written, error_flag, steps).
    `broken`: a block id that never publishes (a producer that died)."""
    rng = random.Random(seed)
    n = n_blocks * BH
    counter = [0] * BH
    written = [[False] * n_blocks for _ in range(BH)]
    next_id, resident, done = 0, [], 0
    bad_read, error, steps = False, False, 0
    while done < n:
        if steps > max_steps:  # no progress: the run is cut off
            return False, bad_read, error, steps
        while len(resident) < slots and next_id < n:  # in-order dispatch
            i, bh = divmod(next_id, BH)
            resident.append({"i": i, "bh": bh, "j": 0, "polls": 0, "id": next_id})
            next_id += 1
        wg = rng.choice(resident)
        steps += 1
        i, bh = wg["i"], wg["bh"]
        if wg["j"] < i:  # waiting for / reading block j
            j = wg["j"]
            if counter[bh] > j:
                bad_read |= not written[bh][j]
                wg["j"] += 1
                wg["polls"] = 0
            else:
                wg["polls"] += 1
                if limit is not None and wg["polls"] > limit:  # bounded wait gives up
                    error = True
                    wg["j"] += 1
                    wg["polls"] = 0
            continue
        # all earlier blocks read: write and publish (unless this producer is broken)
        if wg["id"] != broken:
            written[bh][i] = True
            counter[bh] = max(counter[bh], i + 1)
        resident.remove(wg)
        done += 1
    return True, bad_read, error, steps


@pytest.mark.parametrize("n_blocks,BH,slots", [(16, 1, 1), (16, 4, 3), (32, 8, 8), (64, 2, 5), (12, 16, 64)])
def test_in_order_dispatch_always_finishes_and_never_reads_unpublished(n_blocks, BH, slots):
    """Whatever the interleaving and however few workgroups are resident (one is enough), every
    wait ends without a bound: a workgroup waits only on lower ids, which are resident or done."""
    for seed in range(20):
        finished, bad_read, error, _ = simulate(n_blocks, BH, slots, seed)
        assert finished and not bad_read and not error


def test_bounded_wait_ends_every_workgroup_when_a_producer_never_publishes():
    """A producer that never publishes: unbounded waits would spin forever (the run is cut off),
    bounded waits give up, the error flag is set and every workgroup finishes."""
    finished, _, _, _ = simulate(16, 2, 4, seed=0, broken=10)  # block 5 of head 0
    assert not finished
    finished, _, error, _ = simulate(16, 2, 4, seed=0, limit=50, broken=10)
    assert finished and error
