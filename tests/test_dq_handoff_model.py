"""CPU model of the one-launch backward's dQ hand-over (gpt_amd/csrc/
attn_bwd_fused.hip: the schedule at the end of bwd_fused_d64_kernel and
dq_claim), run under adversarial schedules.

Each workgroup is a generator that yields after every access to the control
block, in the kernel's order: the start mark, one bump per walked block (top
block first, down to its diagonal blocks 2J + 1, 2J), the mailbox close, then
the claim of its own dQ item and of every item posted to it, and the counter
release after running an item. A scheduler admits at most `resident`
workgroups at once, in a random dispatch order, and advances a random resident
one by one access. The model checks what the kernel relies on:

* no deadlock: whatever the residency (down to one workgroup at a time), every
  workgroup ends; a wait is only ever entered while all its contributors have
  started, and those never wait themselves;
* every dQ item runs exactly once, and only after all of its contributions
  have landed (no wait reaches its time limit);
* every launch leaves every counter at 0 and the next launch (next epoch)
  works on the same control block without clearing it.

Start marks are relaxed stores, so the model lets other workgroups see them
late (even after the marked workgroup has closed its mailbox); two planted
mistakes (waiting without the start check, posting to a closed mailbox) show
that the checks catch what they are meant to.
"""
import random

import pytest

CLOSED = 1 << 16
ITEMS = 0xF


class ControlBlock:
    """cnt, mark and mbox words of one (b, h), as the kernel lays them out."""

    def __init__(self, n_kg):
        self.cnt = [0] * n_kg
        self.mark = [0] * n_kg
        self.mbox = [0] * n_kg


def need_of(K, n_qb):
    return (K + 1) * (2 if 2 * K + 1 < n_qb else 1)


def workgroup(J, n_qb, ctl, epoch, log, state):
    """One workgroup of the fused kernel for key group J (a generator)."""
    # start mark: a relaxed store, which other workgroups may see late (the
    # scheduler makes it visible at a random later point, possibly after
    # this workgroup's close)
    state["marks"].append(J)
    yield
    # walk: blocks n_qb - 1 down to 2J; each completed block bumps item i // 2
    for i in range(n_qb - 1, 2 * J - 1, -1):
        ctl.cnt[i >> 1] += 1
        yield
    # close the mailbox (exchange)
    posted = ctl.mbox[J]
    ctl.mbox[J] = (epoch << 32) | CLOSED
    yield
    todo = posted & ITEMS if (posted >> 32) == epoch else 0
    items = [J] + [K for K in range(4) if todo & (1 << K)]
    for K in items:
        need = need_of(K, n_qb)
        run = True
        if K != 0:
            run = yield from claim(K, J, need, ctl, epoch, state)
        if run:
            log.append((K, ctl.cnt[K], need))
            ctl.cnt[K] -= need
            yield


def claim(K, self_j, need, ctl, epoch, state):
    """dq_claim: True = run item K now, False = posted to another key group."""
    c = ctl.cnt[K]
    yield
    if c >= need:
        return True
    for jp in range(K):
        if jp == self_j or state["planted"] == "always_wait":
            continue
        m = ctl.mark[jp]
        yield
        if m == epoch:
            continue
        x = ctl.mbox[jp]
        yield
        while True:
            cur = (x >> 32) == epoch
            if cur and (x & CLOSED) and state["planted"] != "post_to_closed":
                break
            nx = (x if cur else epoch << 32) | (1 << K)
            # compare-and-swap
            if ctl.mbox[jp] == x:
                ctl.mbox[jp] = nx
                state["posts"] += 1
                yield
                return False
            x = ctl.mbox[jp]
            yield
    # every contributor has started: wait (polls; a poll is one access)
    state["waiting"].add(id(state["me"]))
    while True:
        c = ctl.cnt[K]
        yield "poll"
        if c >= need:
            state["waiting"].discard(id(state["me"]))
            return True


def run_launch(n_qb, resident, seed, ctl, epoch, max_events=200000, planted=None):
    rng = random.Random(seed)
    n_kg = (n_qb + 1) // 2
    log = []
    state = {"waiting": set(), "me": None, "posts": 0, "planted": planted, "marks": []}
    order = list(range(n_kg))
    rng.shuffle(order)  # dispatch order: any permutation
    pending = [(J, workgroup(J, n_qb, ctl, epoch, log, state)) for J in order]
    live = []
    events = 0
    polls_in_a_row = 0
    while pending or live:
        while pending and len(live) < resident:
            live.append(pending.pop(0))
        if state["marks"] and rng.random() < 0.05:
            ctl.mark[state["marks"].pop(rng.randrange(len(state["marks"])))] = epoch
        k = rng.randrange(len(live))
        J, g = live[k]
        state["me"] = g
        try:
            r = next(g)
        except StopIteration:
            live.pop(k)
            polls_in_a_row = 0
            continue
        events += 1
        polls_in_a_row = polls_in_a_row + 1 if r == "poll" else 0
        # every resident workgroup stuck polling with nothing else able to move
        assert polls_in_a_row < 50 * max(1, len(live)) + 1000, \
            f"deadlock: n_qb={n_qb} resident={resident} seed={seed} live={[j for j, _ in live]}"
        assert events < max_events, "no progress"
    for J in state["marks"]:
        ctl.mark[J] = epoch
    return log, state["posts"]


@pytest.mark.parametrize("n_qb", [1, 2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("resident", [1, 2, 3, 4])
def test_handover_schedules(n_qb, resident):
    n_kg = (n_qb + 1) // 2
    ctl = ControlBlock(4)
    ctl.mark = [0xdead] * 4  # stale words from an unrelated launch
    ctl.mbox = [(0xbeef << 32) | CLOSED | 0x6] * 4
    for launch in range(60):
        epoch = launch + 1
        log, _ = run_launch(n_qb, resident, seed=1000 * n_qb + 10 * resident + launch, ctl=ctl, epoch=epoch)
        ran = sorted(K for K, _, _ in log)
        assert ran == list(range(n_kg)), f"items run {ran}, expected each of 0..{n_kg - 1} once"
        for K, c, need in log:
            assert c == need, f"item {K} ran with {c} of {need} contributions"
        assert ctl.cnt[:n_kg] == [0] * n_kg


def test_handover_happens_under_low_residency():
    """With few resident workgroups, owners post their items to key groups
    that have not started (the hand-over path is exercised, not just the
    waits)."""
    ctl = ControlBlock(4)
    posts = 0
    for seed in range(200):
        _, p = run_launch(8, 1 + seed % 3, seed, ctl, epoch=seed + 1)
        posts += p
    assert posts > 0


def test_model_catches_a_wait_on_unstarted_work():
    """Planted mistake: owners wait without checking that their contributors
    have started (the earlier whole-grid-resident design). At low residency
    the model finds the deadlock."""
    found = False
    for seed in range(50):
        try:
            run_launch(8, 2, seed, ControlBlock(4), epoch=1, planted="always_wait")
        except AssertionError as e:
            assert "deadlock" in str(e)
            found = True
            break
    assert found


def test_model_catches_a_post_to_a_closed_mailbox():
    """Planted mistake: posting to a mailbox that its owner already closed
    loses the item (it never runs)."""
    lost = False
    for seed in range(300):
        ctl = ControlBlock(4)
        log, _ = run_launch(8, 2 + seed % 3, seed, ctl, epoch=1, planted="post_to_closed")
        if sorted(K for K, _, _ in log) != [0, 1, 2, 3]:
            lost = True
            break
    assert lost
