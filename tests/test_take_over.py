"""The take-over protocol of the one-token FFN's p hand-off, replayed on the host (the device code
is moa_decode.hip: ffn_fused_kernel's claim hook, its p wait and the take-over loop).

Model: a launch of G workgroups over the residual row. Workgroup b owns block b of p; the
leaders rewrite the residual once every block is published. A workgroup reads the residual at
entry (the pre-norm), and p computed from a rewritten residual is wrong. The owner exchanges the
launch's tag into the block's claim word once its norm is done and publishes only if the word did
not already hold the tag; a waiting workgroup that gives up on block b exchanges the same word and
computes the block from its own (unrewritten) normalised row. Random schedules start some owners
late -- after other workgroups have taken their blocks over, and even after the leaders have
rewritten the residual. Every schedule must publish each block exactly once, and only values
computed from the unrewritten residual. The same schedules without the claim (an owner that
always publishes) must fail, which shows that they reach the case the claim exists for."""
import random

import pytest


def run_launch(rng: random.Random, G: int, late: set, use_claim: bool):
    """One launch, event by event. Returns (published[b] list of residual versions used, version)."""
    tag = rng.randrange(1, 2**32)
    claim = {b: rng.randrange(1, 2**32 - 1) for b in range(G)}  # the previous launch's tags
    for b in claim:
        if claim[b] == tag:
            claim[b] += 1
    residual_version = 0          # 0: the launch's input; 1: rewritten by the leaders
    published = {b: [] for b in range(G)}   # versions of the residual each publish was computed from
    # each workgroup's pending steps as a generator, so schedules can interleave them
    def owner(b):
        seen = residual_version                     # the pre-norm reads the residual
        yield
        won = True
        if use_claim:
            old, claim[b] = claim[b], tag           # exchange once the norm is done
            won = old != tag
        yield
        if won:
            published[b].append(seen)

    def taker(b, own_view):
        old, claim[b] = claim[b], tag
        if old != tag:
            published[b].append(own_view)           # computed from the taker's own normalised row
        yield

    active = {b: owner(b) for b in range(G) if b not in late}
    views = {b: 0 for b in range(G) if b not in late}   # resident workgroups read the input version
    late_waiting = sorted(late)
    steps = 0
    while True:
        steps += 1
        assert steps < 100000
        done_all = all(published[b] for b in range(G))
        if done_all and residual_version == 0:
            residual_version = 1                    # the leaders rewrite the residual rows
        # a late owner may start at any point, also after the rewrite
        if late_waiting and rng.random() < 0.2:
            b = late_waiting.pop(rng.randrange(len(late_waiting)))
            active[b] = owner(b)
        if not active and not late_waiting:
            break
        # waiting workgroups take over a missing block now and then (their threshold expired)
        missing = [b for b in range(G) if not published[b]]
        if missing and views and rng.random() < 0.3:
            who = rng.choice(list(views))
            b = rng.choice(missing)
            for _ in taker(b, views[who]):
                pass
        if active:
            b = rng.choice(list(active))
            try:
                next(active[b])
            except StopIteration:
                del active[b]
    return published, residual_version


@pytest.mark.parametrize("seed", range(200))
def test_each_block_published_once_from_the_input_rows(seed):
    rng = random.Random(seed)
    G = rng.choice([4, 8, 16])
    late = set(rng.sample(range(G), rng.randrange(1, G)))
    published, version = run_launch(rng, G, late, use_claim=True)
    assert version == 1, "the launch did not complete"
    for b, pubs in published.items():
        assert len(pubs) == 1, f"block {b} published {len(pubs)} times"
        assert pubs[0] == 0, f"block {b} computed from the rewritten residual"


def test_without_the_claim_a_late_owner_publishes_from_rewritten_rows():
    """The schedules above do reach the dangerous case: without the claim some late owner
    publishes values computed after the rewrite."""
    bad = 0
    for seed in range(200):
        rng = random.Random(seed)
        G = rng.choice([4, 8, 16])
        late = set(rng.sample(range(G), rng.randrange(1, G)))
        published, _ = run_launch(rng, G, late, use_claim=False)
        bad += any(1 in pubs for pubs in published.values())
    assert bad > 0
