"""Host model of the statistics-exchange protocol of the GroupNorm kernels
(k_norm.hip k_gn_nchw_xchg, k_gemm.hip k_splitk_reduce_gn with NS > 1; the
record layout and rules are in di_device.h): per group record, NS slots of
64-bit words {epoch, value} and a 32-bit arrival counter.  A workgroup
fetch-adds the counter (o), publishes its value under epoch o // NS + 1 and
accepts the record once every slot carries that epoch.

The model runs launches one after another on one stream (as the context's
launches are), each with NS workgroups per group in a random interleaving,
stores that become visible to other workgroups only after a random delay,
and launches over different group counts.  It checks the property the
kernels rely on: a workgroup that accepts a record sees exactly the values
its own launch published (never a stale word), and every workgroup of a
launch derives the same epoch.  It also checks that the counter, wrapping
at 2^32, keeps launches aligned when NS divides 2^32.
"""
import random

import pytest


class Record:
    def __init__(self, ns):
        self.ns = ns
        self.counter = 0          # 32-bit arrival counter
        self.words = [(0, None)] * ns  # globally visible (epoch, value)
        self.pending = []         # (visible_at_step, slot, word)


def run_launch(recs, groups, ns, rng, step0, max_delay, values,
               epoch_of=lambda o, ns: (o // ns + 1) % (1 << 32)):
    """One launch over `groups` records.  Returns the accepted values per
    (group, slice) and the epochs the workgroups derived."""
    wgs = [(g, s) for g in range(groups) for s in range(ns)]
    state = {w: "arrive" for w in wgs}
    epoch = {}
    accepted = {}
    step = step0
    while any(v != "done" for v in state.values()):
        step += 1
        # stores become visible in their own time
        for r in recs[:groups]:
            keep = []
            for t, slot, word in r.pending:
                if t <= step:
                    r.words[slot] = word
                else:
                    keep.append((t, slot, word))
            r.pending = keep
        w = rng.choice([w for w in wgs if state[w] != "done"])
        g, s = w
        r = recs[g]
        if state[w] == "arrive":
            o = r.counter
            r.counter = (r.counter + 1) % (1 << 32)
            epoch[w] = epoch_of(o, ns)
            state[w] = "publish"
        elif state[w] == "publish":
            r.pending.append((step + rng.randint(0, max_delay), s, (epoch[w], values[w])))
            state[w] = "poll"
        else:
            if all(word[0] == epoch[w] for word in r.words):
                accepted[w] = [word[1] for word in r.words]
                state[w] = "done"
    # drain the stores (the launch ends only when its writes are complete)
    for r in recs[:groups]:
        for _, slot, word in r.pending:
            r.words[slot] = word
        r.pending = []
    return accepted, epoch, step


@pytest.mark.parametrize("ns", [4, 8])
def test_never_accepts_stale_words(ns):
    rng = random.Random(1234 + ns)
    max_groups = 6
    recs = [Record(ns) for _ in range(max_groups)]
    step = 0
    for launch in range(60):
        groups = rng.randint(1, max_groups)  # launches over different group counts
        values = {(g, s): (launch, g, s, rng.random()) for g in range(groups) for s in range(ns)}
        accepted, epoch, step = run_launch(recs, groups, ns, rng, step, rng.randint(0, 12), values)
        for g in range(groups):
            eps = {epoch[(g, s)] for s in range(ns)}
            assert len(eps) == 1, "the workgroups of one launch derive one epoch per record"
            want = [values[(g, s)] for s in range(ns)]
            for s in range(ns):
                assert accepted[(g, s)] == want, "accepted a word of another launch"


def test_planted_epoch_without_offset_is_caught():
    """The model is sensitive: an epoch of o // NS (the +1 dropped) makes the
    first launch's epoch that of the zeroed records, so a workgroup polling
    before its peers' words land accepts the zeros."""
    rng = random.Random(11)
    ns = 8
    caught = False
    for trial in range(20):
        recs = [Record(ns)]
        values = {(0, s): (trial, s) for s in range(ns)}
        accepted, _, _ = run_launch(recs, 1, ns, rng, 0, 10, values, epoch_of=lambda o, n: o // n)
        caught |= any(accepted[(0, s)] != [values[(0, j)] for j in range(ns)] for s in range(ns))
    assert caught


def test_planted_misalignment_is_caught():
    """The model is sensitive: a launch that adds one arrival too few to a
    record (a counter no longer a multiple of NS at a launch's start) splits
    the next launch's workgroups over two epochs."""
    ns = 8
    rec = Record(ns)
    rec.counter = 8 * 5 + 7  # one arrival short of a whole launch
    epochs = set()
    for _ in range(ns):
        o = rec.counter
        rec.counter += 1
        epochs.add(o // ns + 1)
    assert len(epochs) == 2


@pytest.mark.parametrize("ns", [4, 8])
def test_counter_wrap_keeps_launches_aligned(ns):
    """Launches that straddle the 32-bit wrap of the counter: NS divides
    2^32, so each launch's workgroups still share one epoch, and it differs
    from the previous launch's."""
    top = 1 << 32
    counter = top - 3 * ns  # three launches before the wrap
    prev = None
    for _ in range(6):
        eps = set()
        for _ in range(ns):
            eps.add((counter // ns + 1) % top)
            counter = (counter + 1) % top
        assert len(eps) == 1
        (e,) = eps
        assert e != prev and e != 0  # 0 is the zeroed record's epoch: never valid
        prev = e
