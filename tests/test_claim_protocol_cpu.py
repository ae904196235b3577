"""A CPU replay of the work-claiming protocols of the persistent attention
kernels (attend_step_bf16_kernel with leave_and_reset, and attend_tile_kernel
with its last-claim reset, csrc/attention.hip):
workgroups as coroutines that interleave their atomic operations in random
orders. Each kernel's counters are touched only by atomic operations on
single words, so any interleaving of those operations is a possible
execution; the replay checks, over many random ones and back-to-back
launches of different shapes:

  * every item of every queue is run exactly once and no item index at or
    past its queue's length reaches an item body (the bodies index the plan's
    arrays with it);
  * the counters are all zero again when a launch ends (the last workgroup to
    leave resets them; in the tile kernel, the claim that returns the
    queue's last value), so the next launch starts from zero without a
    memset.
"""

import random

XCDS = 8


def step_workgroup(b, grid, n_dec, n_tiles, ctr, ran, tile_first_every=2):
    """attend_step_bf16_kernel's claim loop for workgroup b; yields at every
    atomic operation on the counters (ctr[0] decode queue, ctr[1 + x] tile
    queue x, ctr[9] workgroups finished)."""
    xcd = b % XCDS
    tiles_first = (b // XCDS) % tile_first_every == 0
    for v in range(XCDS + 1):
        if tiles_first:
            qid = 1 + (xcd + v) % XCDS if v < XCDS else 0
        else:
            qid = 0 if v == 0 else 1 + (xcd + v - 1) % XCDS
        tiles = qid != 0
        stride, base = (XCDS, qid - 1) if tiles else (1, 0)
        n = n_tiles if tiles else n_dec
        yield
        seen = ctr[qid]  # an atomic load
        if seen * stride + base >= n:
            continue
        yield
        claim = ctr[qid]
        ctr[qid] += 1  # atomicAdd
        it = claim * stride + base
        while it < n:
            yield
            nxt = ctr[qid]
            ctr[qid] += 1  # the next item, claimed before this one runs
            assert 0 <= it < n
            ran.append((qid == 0, it))
            it = nxt * stride + base
    # leave_and_reset(counters, 9)
    yield
    prev = ctr[9]
    ctr[9] += 1
    if prev == grid - 1:
        for k in range(10):
            yield
            ctr[k] = 0


def run_launch(rng, grid, n_dec, n_tiles, ctr):
    ran = []
    live = [step_workgroup(b, grid, n_dec, n_tiles, ctr, ran) for b in range(grid)]
    while live:
        g = rng.choice(live)
        try:
            next(g)
        except StopIteration:
            live.remove(g)
    return ran


def test_every_item_runs_once_and_counters_return_to_zero():
    rng = random.Random(0)
    ctr = [0] * 10
    for trial in range(300):
        grid = rng.choice([1, 2, 8, 9, 16, 24, 64])
        n_dec = rng.choice([0, 1, 5, 8, 40, 200])
        n_tiles = rng.choice([0, 1, 7, 8, 16, 33, 96])
        ran = run_launch(rng, grid, n_dec, n_tiles, ctr)
        dec = sorted(it for d, it in ran if d)
        til = sorted(it for d, it in ran if not d)
        assert dec == list(range(n_dec)), (trial, grid, n_dec)
        assert til == list(range(n_tiles)), (trial, grid, n_tiles)
        assert ctr == [0] * 10, (trial, ctr)


def test_a_launch_without_its_reset_would_skip_items():
    """The check above has teeth: counters left non-zero by a launch that did
    not reset them make the next launch skip items (never run one twice or
    past its queue: the claim bound holds against any start value)."""
    rng = random.Random(1)
    ctr = [0] * 10
    ctr[0] = 3  # a stale decode counter
    ran = run_launch(rng, 8, 10, 0, ctr)
    dec = sorted(it for d, it in ran if d)
    assert dec == list(range(3, 10))


def tile_workgroup(b, grid, n_items, ctr, ran):
    """attend_tile_kernel's claim loop for workgroup b: queue x = b % 8 holds
    items x, x + 8, ... below n_items; workgroup b starts on item
    (b // 8) * 8 + x, claims the next before running the current one, and the
    claimer whose claim returns the queue's last value (its item count - 1)
    zeroes the queue's counter. Yields at every atomic operation."""
    xcd = b % XCDS
    per_queue = (grid + XCDS - 1 - xcd) // XCDS
    n_q = (n_items - xcd + XCDS - 1) // XCDS if n_items > xcd else 0
    it = (b // XCDS) * XCDS + xcd
    while it < n_items:
        yield
        c = ctr[xcd]
        ctr[xcd] += 1  # atomicAdd
        if c == n_q - 1:
            yield
            ctr[xcd] = 0  # atomic store
        c64 = per_queue + c
        nxt = n_items if c64 < 0 or c64 * XCDS + xcd >= n_items else c64 * XCDS + xcd
        assert 0 <= it < n_items
        ran.append(it)
        it = nxt


def test_tile_queues_run_every_item_once_and_reset_on_the_last_claim():
    rng = random.Random(2)
    ctr = [0] * XCDS
    for trial in range(400):
        grid = rng.choice([8, 9, 16, 24, 64, 96])
        n_items = rng.choice([0, 1, 5, 8, 9, 40, 200, 777])
        ran = []
        live = [tile_workgroup(b, grid, n_items, ctr, ran) for b in range(grid)]
        while live:
            g = rng.choice(live)
            try:
                next(g)
            except StopIteration:
                live.remove(g)
        assert sorted(ran) == list(range(n_items)), (trial, grid, n_items)
        assert ctr == [0] * XCDS, (trial, grid, n_items, ctr)
